"""Host-side choice of the prefill GEMM (no GPU): linear_dequantized takes the library's split-K GEMM only for the
shapes where it measured faster than hipBLASLt (K >= 8192 at 128-768 tokens) and only for BF16 GPU tensors it can
address; NWC_GEMM overrides the choice."""
import pytest
import torch

import nwc_amd.nwc_torch as N


@pytest.mark.parametrize("tokens,out_f,in_f,want", [
    (512, 2560, 9728, True),       # Qwen3-4B down
    (128, 2560, 9728, True),
    (768, 2560, 9728, True),
    (64, 2560, 9728, False),       # too few tokens
    (1024, 2560, 9728, False),     # enough tiles for hipBLASLt
    (512, 2560, 4096, False),      # o: hipBLASLt faster
    (512, 6144, 2560, False),      # qkv
    (512, 19456, 2560, False),     # gate_up
])
def test_gemm_preferred(tokens, out_f, in_f, want):
    assert N.gemm_preferred(tokens, out_f, in_f) is want


def test_gemm_usable_needs_bf16_gpu_rows_of_16_bytes():
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    w = torch.zeros(8, 128, dtype=torch.bfloat16)
    assert not N.gemm_usable(x, w)                       # CPU tensors
    assert not N.gemm_usable(x.float(), w.float())


def test_cpu_tensors_take_f_linear(monkeypatch):
    """Off the GPU the helper is F.linear itself, whatever NWC_GEMM says (the library GEMM needs device pointers)."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 512, generator=g).to(torch.bfloat16)
    w = torch.randn(16, 512, generator=g).to(torch.bfloat16)
    b = torch.randn(16, generator=g).to(torch.bfloat16)
    for mode in ("auto", "nwc", "hipblaslt"):
        monkeypatch.setattr(N, "GEMM", mode)
        assert torch.equal(N.linear_dequantized(x, w, b), torch.nn.functional.linear(x, w, b))
