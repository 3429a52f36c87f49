"""GPU tests of the Python API over the C ABI: NWCLinear's token path (fused kernel) and prefill path (decompression
+ hipBLASLt), weight-only fp8, NWCEmbedding (gather kernel), fuse/convert on a random-init Qwen3-shaped model,
and the checkpoint round trip with logits compared bit for bit (reference tests/test_nwc_torch.py,
tests/test_checkpoint.py:28-56, tests/test_fp8.py).

Bars: token path rounded to nearest even from within 1e-3 |y| + 1e-5 of a float64 matvec on the decoded weights; 2-8 tokens of a layout-0
matrix (the batched kernel) equal, token by token, to the single-token path; prefill (more tokens, or another layout)
equal to F.linear on the original weights (the same GEMM on bit-identical operands); decoded weights and gathered rows
bit-exact;
model logits within 5% of the logit range of the uncompressed model (the reference doctor's bar, doctor.py:83)
and bit-identical between a converted model and its reloaded checkpoint."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.helpers import bf16_matrix, bits16, check_rne, fp8_source, ref_matvec64, token_tol

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
    check_rne(y1, y64, token_tol(y64))
    x5 = torch.randn(1, 5, K, generator=g).to(torch.bfloat16).cuda()
    y5 = lin(x5)
    if layout == 0:                         # the batched kernel: each token as the single-token path computes it
        assert torch.equal(y5, torch.cat([lin(x5[:, t:t + 1]) for t in range(5)], dim=1))
    else:                                   # decompression + F.linear
        assert torch.equal(y5, F.linear(x5, w.cuda(), b.cuda()))
    x12 = torch.randn(1, 12, K, generator=g).to(torch.bfloat16).cuda()
    assert torch.equal(lin(x12), F.linear(x12, w.cuda(), b.cuda()))


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
    check_rne(lin(x1), y64, token_tol(y64))
    x3 = torch.randn(3, K, generator=g).to(torch.bfloat16).cuda()
    if layout == 0:                         # the batched kernel: each token as the single-token path computes it
        assert torch.equal(lin(x3), torch.cat([lin(x3[t:t + 1]) for t in range(3)]))
    x12 = torch.randn(12, K, generator=g).to(torch.bfloat16).cuda()
    want = (F.linear(x12, q.to(torch.bfloat16).cuda()).float() * scale.cuda()).to(torch.bfloat16)
    assert torch.equal(lin(x12), want)


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
    check_rne(mod(x), y64, token_tol(y64))


def test_qwen2_checkpoint_round_trip_with_fp8(cuda, tmp_path):
    """The reference's tests/test_checkpoint.py flow on its tiny random Qwen2 (vocab 4096, hidden 256, intermediate 1000,
    2 layers, tied embeddings; projection biases on q/k/v, a down_proj with K = 1000 not a multiple of 16): fuse +
    convert -> save -> load gives identical logits; export_bf16 gives every original tensor back bit for bit and a
    model whose logits equal the original's; an fp8 conversion of the exported model reproduces its logits after
    save -> load (test_checkpoint.py:11-56)."""
    import nwc_amd
    from safetensors.torch import load_file
    from transformers import AutoModelForCausalLM, Qwen2Config
    print("tiny Qwen2 checkpoint round trip", flush=True)
    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=4096, hidden_size=256, intermediate_size=1000, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, max_position_embeddings=512, tie_word_embeddings=True)
    try:
        model = AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16).eval()
    except TypeError:
        model = AutoModelForCausalLM.from_config(cfg, torch_dtype=torch.bfloat16).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, 12), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        ref = model(ids).logits.float()                                     # BF16 on the CPU
    state = {k: v.clone() for k, v in model.state_dict().items()}
    nwc_amd.fuse(model, device="cuda")
    nwc_amd.convert(model, device="cuda", verbose=False)
    with torch.no_grad():
        a = model(ids.cuda()).logits.float()
    d = tmp_path / "ckpt"
    c = nwc_amd.save_pretrained(model, str(d), base_model="test")
    assert c["bytes_nwc"] < c["bytes_bf16"] and len(c["weights"]) > 0
    del model
    m2 = nwc_amd.load_pretrained(str(d), device="cuda", verbose=False)
    with torch.no_grad():
        b = m2(ids.cuda()).logits.float()
    assert torch.equal(a, b)
    assert (b.cpu() - ref).abs().max() < 0.5
    assert all(p.device.type == "cuda" for p in m2.parameters())
    e = tmp_path / "bf16"
    nwc_amd.export_bf16(str(d), str(e), device="cuda", verbose=False)
    exported = load_file(str(e / "model.safetensors"))
    missing = [k for k in state if k not in exported and k != "lm_head.weight"]
    differ = [k for k in state if k in exported and not torch.equal(exported[k].to(state[k].dtype), state[k])]
    assert not missing and not differ, (missing[:3], differ[:3])
    try:
        m3 = AutoModelForCausalLM.from_pretrained(str(e), dtype=torch.bfloat16).eval()
    except TypeError:
        m3 = AutoModelForCausalLM.from_pretrained(str(e), torch_dtype=torch.bfloat16).eval()
    with torch.no_grad():
        assert torch.equal(m3(ids).logits.float(), ref)
    nwc_amd.fuse(m3, device="cuda", elem="fp8")
    nwc_amd.convert(m3, device="cuda", verbose=False, elem="fp8")
    with torch.no_grad():
        a8 = m3(ids.cuda()).logits.float()
    nwc_amd.save_pretrained(m3, str(tmp_path / "fp8"), base_model="test")
    del m3
    m5 = nwc_amd.load_pretrained(str(tmp_path / "fp8"), device="cuda", verbose=False)
    with torch.no_grad():
        assert torch.equal(m5(ids.cuda()).logits.float(), a8)
