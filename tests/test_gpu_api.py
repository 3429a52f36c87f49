"""GPU tests of the Python API over the C ABI: NWCLinear's token path (fused kernel) and prefill path (decompression
+ hipBLASLt), weight-only fp8, NWCEmbedding (gather kernel), fuse/convert on a random-init Qwen3-shaped model,
and the checkpoint round trip with logits compared bit for bit (reference tests/test_nwc_torch.py,
tests/test_checkpoint.py:28-56, tests/test_fp8.py).

Bars: token path within one BF16 ulp of a float64 matvec on the decoded weights (+1e-5); prefill equal to F.linear
on the original weights (the same GEMM on bit-identical operands); decoded weights and gathered rows bit-exact;
model logits within 5% of the logit range of the uncompressed model (the reference doctor's bar, doctor.py:83)
and bit-identical between a converted model and its reloaded checkpoint."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.helpers import bf16_matrix, bits16, fp8_source, ref_matvec64

pytestmark = pytest.mark.gpu


def tiny_qwen3(tied=False, seed=0):
    """Built the way load_pretrained builds a model (from_config in BF16), so both keep the rotary inverse
    frequencies in fp32 and their logits can be compared bit for bit."""
    from transformers import AutoModelForCausalLM, Qwen3Config
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=64, tie_word_embeddings=tied)
    torch.manual_seed(seed)
    try:
        model = AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16)
    except TypeError:
        model = AutoModelForCausalLM.from_config(cfg, torch_dtype=torch.bfloat16)
    return model.eval()


@pytest.mark.parametrize("layout", [0, 1, 2])
def test_nwclinear_token_and_prefill(cuda, layout):
    from nwc_amd.nwc_torch import NWCLinear, NWCWeight
    M, K = 300, 1000
    print(f"NWCLinear layout {layout}", flush=True)
    w = bf16_matrix(M, K, seed=3, escapes=False)
    g = torch.Generator().manual_seed(4)
    b = (torch.rand(M, generator=g) - 0.5).to(torch.bfloat16)
    lin = NWCLinear(w=NWCWeight(w, device="cuda", layout=layout), bias=b, device="cuda")
    x1 = torch.randn(1, 1, K, generator=g).to(torch.bfloat16).cuda()
    y1 = lin(x1)
    assert y1.shape == (1, 1, M) and y1.dtype == torch.bfloat16
    y64 = ref_matvec64(bits16(w), x1.float().cpu().numpy().ravel(), bias_bits=bits16(b))
    err = np.abs(y1.double().cpu().numpy().ravel() - y64)
    assert np.all(err <= 2.0 ** -8 * np.abs(y64) + 1e-5)
    x5 = torch.randn(1, 5, K, generator=g).to(torch.bfloat16).cuda()
    assert torch.equal(lin(x5), F.linear(x5, w.cuda(), b.cuda()))


@pytest.mark.parametrize("layout", [0, 1])
def test_nwclinear_fp8(cuda, layout):
    from nwc_amd.nwc_torch import NWCLinear, NWCWeight, quantize_fp8
    M, K = 257, 1024
    w = fp8_source(M, K, seed=9)
    q, scale = quantize_fp8(w)
    lin = NWCLinear(w=NWCWeight(w, device="cuda", elem="fp8", layout=layout), device="cuda")
    g = torch.Generator().manual_seed(5)
    x1 = torch.randn(1, K, generator=g).to(torch.bfloat16).cuda()
    y64 = ref_matvec64(bits16(q.to(torch.bfloat16)), x1.float().cpu().numpy().ravel(), scale=scale.numpy())
    err = np.abs(lin(x1).double().cpu().numpy().ravel() - y64)
    assert np.all(err <= 2.0 ** -8 * np.abs(y64) + 1e-5)
    x3 = torch.randn(3, K, generator=g).to(torch.bfloat16).cuda()
    want = (F.linear(x3, q.to(torch.bfloat16).cuda()).float() * scale.cuda()).to(torch.bfloat16)
    assert torch.equal(lin(x3), want)


def test_embedding_gather(cuda):
    from nwc_amd.nwc_torch import NWCEmbedding, NWCWeight
    w = bf16_matrix(1000, 384, seed=12, escapes=False)
    emb = NWCEmbedding(w=NWCWeight(w, device="cuda"), padding_idx=None)
    ids = torch.tensor([[0, 999, 5, 5, 512], [7, 1, 2, 3, 4]], device="cuda")
    out = emb(ids)
    assert out.shape == (2, 5, 384)
    assert torch.equal(out.cpu().view(torch.int16), w[ids.cpu()].view(torch.int16))


def _logits(model, ids):
    with torch.no_grad():
        return model(input_ids=ids).logits.float()


def _close(a, b):
    return (a - b).abs().max().item() <= 0.05 * (b.max() - b.min()).item()


@pytest.mark.parametrize("tied", [False, True])
def test_model_convert_generate_and_checkpoint(cuda, tmp_path, tied):
    import nwc_amd
    print(f"tiny Qwen3 tied={tied}", flush=True)
    ref = tiny_qwen3(tied=tied).cuda()
    orig = {n: p.detach().clone().cpu() for n, p in ref.named_parameters()}
    ids = torch.randint(0, 512, (1, 12), generator=torch.Generator().manual_seed(1)).cuda()
    want = _logits(ref, ids)
    # one decode step after the prompt (token path) on the uncompressed model
    with torch.no_grad():
        out = ref(input_ids=ids, use_cache=True)
        nxt = out.logits[:, -1:].argmax(-1)
        want_step = ref(input_ids=nxt, past_key_values=out.past_key_values, use_cache=True).logits.float()

    model = tiny_qwen3(tied=tied)
    nwc_amd.fuse(model, device="cuda")
    nwc_amd.convert(model, device="cuda", verbose=False)
    got = _logits(model, ids)                                   # prefill: decompression + hipBLASLt
    assert _close(got, want)
    with torch.no_grad():
        out = model(input_ids=ids, use_cache=True)
        got_step = model(input_ids=nxt, past_key_values=out.past_key_values, use_cache=True).logits.float()
    assert _close(got_step, want_step)                          # token path: fused decode-matvec kernels

    nwc_amd.save_pretrained(model, str(tmp_path / "ckpt"))
    loaded = nwc_amd.load_pretrained(str(tmp_path / "ckpt"), device="cuda", verbose=False)
    assert torch.equal(_logits(loaded, ids), got)
    with torch.no_grad():
        out2 = loaded(input_ids=ids, use_cache=True)
        step2 = loaded(input_ids=nxt, past_key_values=out2.past_key_values, use_cache=True).logits.float()
    assert torch.equal(step2, got_step)

    from safetensors.torch import load_file
    nwc_amd.export_bf16(str(tmp_path / "ckpt"), str(tmp_path / "bf16"), device="cuda", verbose=False)
    exported = load_file(str(tmp_path / "bf16" / "model.safetensors"))
    for n, p in orig.items():
        if n in exported:
            assert torch.equal(exported[n].view(torch.int16), p.view(torch.int16)), n
    assert all(f"model.layers.{i}.mlp.gate_proj.weight" in exported for i in range(2))


def test_ref_fp8_baseline_module(cuda):
    from nwc_amd.nwc_torch import RefFP8Linear, quantize_fp8
    import torch.nn as nn
    M, K = 200, 768
    w = fp8_source(M, K, seed=21)
    lin = nn.Linear(K, M, bias=False, dtype=torch.bfloat16)
    lin.weight.data = w
    mod = RefFP8Linear(lin, device="cuda")
    q, scale = quantize_fp8(w)
    x = torch.randn(1, K, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    y64 = ref_matvec64(bits16(q.to(torch.bfloat16)), x.float().cpu().numpy().ravel(), scale=scale.numpy())
    err = np.abs(mod(x).double().cpu().numpy().ravel() - y64)
    assert np.all(err <= 2.0 ** -8 * np.abs(y64) + 1e-5)
