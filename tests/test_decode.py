"""Model-level batch-1 decode (bench.py --decode): the attention used there, the static-cache greedy loop, and on the
GPU, HIP-graph replays of a converted model's token step against eager steps (bit for bit) — the reference's
scripts/graph_decode.py:40-67 flow on a tiny random-init Qwen3."""
import pytest
import torch

import bench


def _tiny(vocab=512):
    return dict(vocab_size=vocab, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                num_key_value_heads=2, head_dim=64)


def test_contiguous_attention_matches_eager_cpu():
    model = bench.qwen3_model(_tiny(), seed=3, device="cpu")
    ids = torch.randint(0, 512, (1, 10), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        got = model(input_ids=ids).logits.float()
        model.config._attn_implementation = "eager"
        for layer in model.model.layers:
            layer.self_attn.config._attn_implementation = "eager"
        want = model(input_ids=ids).logits.float()
    # eager attention rounds its softmax to BF16 before the value product; this one keeps fp32
    assert (got - want).abs().max() < 0.05 * want.abs().max()


def test_static_cache_greedy_loop_cpu():
    """GraphDecoder's prefill + steps (no graph) give the same tokens and logits as a plain forward over the growing
    sequence."""
    model = bench.qwen3_model(_tiny(), seed=5, device="cpu")
    ids = torch.randint(0, 512, (1, 6), generator=torch.Generator().manual_seed(6))
    d = bench.GraphDecoder(model, ids, 8)
    d.prefill()
    seq = ids
    for i in range(4):
        d.step()
        seq = torch.cat([seq, d.res[i:i + 1].view(1, 1)], dim=1)
        with torch.no_grad():
            full = model(input_ids=seq).logits[0, -1].float()
        assert int(full.argmax()) == int(d.res[i + 1])
        assert (full - d.logits).abs().max() < 0.05 * full.abs().max()      # BF16 rounding of other row counts


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["nwc", "bf16"])
def test_graph_decode_replays_equal_eager(cuda, mode):
    """Qwen3's 151936-token vocabulary, so the greedy token comes from a large argmax; "bf16" keeps the uncompressed
    model (torch embedding lookup, hipBLASLt linears)."""
    import nwc_amd
    print(f"tiny Qwen3 graph decode, {mode}", flush=True)
    model = bench.qwen3_model(_tiny(vocab=151936), seed=8, device="cuda")
    if mode == "nwc":
        nwc_amd.fuse(model, device="cuda")
        nwc_amd.convert(model, device="cuda", verbose=False)
    ids = torch.randint(0, 151936, (1, 12), generator=torch.Generator().manual_seed(9)).cuda()
    d = bench.GraphDecoder(model, ids, 16)
    d.prefill()
    eager = []
    for _ in range(6):
        d.step()
        eager.append(d.logits.clone())
    tokens = d.res[:7].clone()
    d.capture()
    d.prefill()
    for i in range(6):
        d.graph.replay()
        torch.cuda.synchronize()
        x = torch.randn(64, device="cuda").sum()                 # eager work between replays
        assert torch.equal(d.logits, eager[i]), f"replay {i}"
    assert torch.equal(d.res[:7], tokens)


def test_contiguous_attention_with_static_cache_cpu():
    """Prefill and decode steps through a static cache (boolean masks over the cache length) agree with eager
    attention without a cache."""
    from transformers import StaticCache
    model = bench.qwen3_model(_tiny(), seed=11, device="cpu")
    ids = torch.randint(0, 512, (1, 7), generator=torch.Generator().manual_seed(12))
    cache = StaticCache(config=model.config, max_cache_len=24)
    with torch.no_grad():
        got = [model(input_ids=ids, past_key_values=cache, cache_position=torch.arange(7), use_cache=True).logits[0, -1]]
        nxt = torch.tensor([[3]])
        got.append(model(input_ids=nxt, past_key_values=cache, cache_position=torch.tensor([7]), use_cache=True).logits[0, -1])
        model.config._attn_implementation = "eager"
        for layer in model.model.layers:
            layer.self_attn.config._attn_implementation = "eager"
        want = [model(input_ids=ids).logits[0, -1], model(input_ids=torch.cat([ids, nxt], 1)).logits[0, -1]]
    for g, w in zip(got, want):
        assert (g.float() - w.float()).abs().max() < 0.05 * w.float().abs().max()


def test_greedy_token_is_first_argmax_cpu():
    g = torch.Generator().manual_seed(13)
    for n in (1, 7, 128, 512, 1000, 151936):
        x = torch.randn(n, generator=g)
        assert int(bench.greedy_token(x)) == int(x.argmax())
        x = torch.zeros(n)                                  # ties: the first index, as torch.argmax
        x[n // 3] = 1.0
        x[n - 1] = 1.0
        assert int(bench.greedy_token(x)) == int(x.argmax()) == n // 3 if n > 1 else True
    x = torch.randint(0, 3, (151936,), generator=g).float()
    assert int(bench.greedy_token(x)) == int(x.argmax())


@pytest.mark.gpu
def test_graph_decode_nwc_matches_bf16_model(cuda):
    """The converted model's HIP-graph decode against the uncompressed model's, both greedy from the same prompt on a
    4-layer random-init Qwen3 with the Qwen3-0.6B layer shapes (hidden 1024, intermediate 3072, 16 heads, 8 KV heads)
    and the 151936-token tied vocabulary.  The weights are bit-identical (lossless BF16); only the token path's
    summation order differs from hipBLASLt's.  While the two token sequences agree, every step's logits must agree to
    5% of their range, and the greedy token must agree wherever the uncompressed model's top-two margin exceeds twice
    the largest logit difference seen so far."""
    import nwc_amd
    print("Qwen3-0.6B-shaped 4-layer graph decode, nwc vs bf16", flush=True)
    cfg = dict(bench.QWEN3_ARCH["qwen3-0.6b"], num_hidden_layers=4)
    ids = torch.randint(0, 151936, (1, 16), generator=torch.Generator().manual_seed(21)).cuda()
    runs = {}
    for mode in ("bf16", "nwc"):
        model = bench.qwen3_model(cfg, seed=17, device="cuda")
        if mode == "nwc":
            nwc_amd.fuse(model, device="cuda")
            nwc_amd.convert(model, device="cuda", verbose=False)
        d = bench.GraphDecoder(model, ids, 24)
        d.capture()
        d.prefill()
        logits = [d.logits.clone()]
        for _ in range(24):
            d.graph.replay()
            logits.append(d.logits.clone())
        torch.cuda.synchronize()
        runs[mode] = (torch.stack(logits).cpu(), d.res[:25].cpu())
        del d, model
        torch.cuda.empty_cache()
    (lb, tb), (ln, tn) = runs["bf16"], runs["nwc"]
    worst = 0.0
    for i in range(25):
        if i > 0 and not torch.equal(tb[:i], tn[:i]):
            break                                                 # the sequences differ from here on
        diff = (ln[i] - lb[i]).abs().max().item()
        worst = max(worst, diff)
        assert diff <= 0.05 * (lb[i].max() - lb[i].min()).item(), f"step {i}"
        top2 = lb[i].topk(2).values
        if (top2[0] - top2[1]).item() > 2 * worst:
            assert int(tn[i]) == int(tb[i]), f"step {i}"
    print(f"steps compared: {i + 1 if torch.equal(tb, tn) else i}, largest logit difference {worst:.4f}", flush=True)
