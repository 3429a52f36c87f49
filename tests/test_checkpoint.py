"""Checkpoint round trip on the CPU (reference tests/test_checkpoint.py, whose GPU half lives in
tests/test_gpu_api.py): a random-init Qwen3-shaped model is fused and converted, saved with save_pretrained and
loaded with load_pretrained.  Every stored tensor must come back bit-identical, the compressed matrices must decode
(oracle) to the original BF16 weights, and the files must follow the reference layout (nwc_config.json keys,
"nwc/<id>/<tensor>" names, checkpoint.py:1-16)."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits16, oracle_encoding


def tiny_qwen3(tied=False, seed=0):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=512, hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=16, tie_word_embeddings=tied)
    torch.manual_seed(seed)
    return Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()


def _originals(model):
    return {n: p.detach().clone() for n, p in model.named_parameters()}


@pytest.mark.parametrize("tied", [False, True])
def test_save_load_roundtrip_cpu(tmp_path, tied):
    import nwc_amd
    from nwc_amd.nwc_torch import NWCEmbedding, NWCLinear
    model = tiny_qwen3(tied=tied)
    orig = _originals(model)
    nwc_amd.fuse(model, device="cpu")
    nwc_amd.convert(model, device="cpu", verbose=False)
    cfg = nwc_amd.save_pretrained(model, str(tmp_path))
    files = set(os.listdir(tmp_path))
    assert {"config.json", "nwc_config.json", "model.safetensors"} <= files
    meta = json.load(open(tmp_path / "nwc_config.json"))
    assert meta["nwc_checkpoint"] == 1 and meta["library_version"] == 11
    assert {m["kind"] for m in meta["modules"]} >= {"fused", "linear", "embedding"}

    loaded = nwc_amd.load_pretrained(str(tmp_path), device="cpu", verbose=False)
    # every compressed matrix: identical tensors, and the oracle decodes them to the original weights
    mods = dict(model.named_modules())
    for path, m in loaded.named_modules():
        if isinstance(m, (NWCLinear, NWCEmbedding)):
            a, b = m.w, mods[path].w
            for t in ("data", "bases", "hdr", "lut", "low"):
                assert torch.equal(getattr(a, t), getattr(b, t)), f"{path}.{t}"
            dec = O.decode(oracle_encoding(a)).reshape(a.out_features, a.in_features)
            key = path + ".weight"
            if key in orig:
                assert np.array_equal(dec, bits16(orig[key]))
    # the fused groups decode to the concatenated originals
    for i in range(2):
        for names, parent in ((("q_proj", "k_proj", "v_proj"), f"model.layers.{i}.self_attn"),
                              (("gate_proj", "up_proj"), f"model.layers.{i}.mlp")):
            head = loaded.get_submodule(f"{parent}.{names[0]}")
            w = head.group.lin.w
            dec = O.decode(oracle_encoding(w)).reshape(w.out_features, w.in_features)
            want = torch.cat([orig[f"{parent}.{n}.weight"] for n in names], 0)
            assert np.array_equal(dec, bits16(want))
    # the uncompressed parameters (norms) come back unchanged
    lp = dict(loaded.named_parameters())
    for n, p in orig.items():
        if "norm" in n:
            assert torch.equal(lp[n].cpu(), p)
    assert cfg["bytes_bf16"] == sum(2 * e["out"] * e["in"] for e in meta["weights"])


def test_incompatible_version_rejected(tmp_path):
    import nwc_amd
    model = tiny_qwen3()
    nwc_amd.convert(model, device="cpu", verbose=False)
    nwc_amd.save_pretrained(model, str(tmp_path))
    meta = json.load(open(tmp_path / "nwc_config.json"))
    meta["library_version"] = 8
    json.dump(meta, open(tmp_path / "nwc_config.json", "w"))
    with pytest.raises(RuntimeError):
        nwc_amd.load_pretrained(str(tmp_path), device="cpu", verbose=False)
