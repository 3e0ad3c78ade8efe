"""The two largest workloads at their full sizes, against the oracle.

* The 12-layer forward at T=16384 (B=1, bf16, N(0, 0.02) weights, RMSNorm eps
  1e-5, block 64, top-8), layer L's forecast routing layer L+1
  (model/model.py:97-139). Past 8192 tokens every layer takes the chunked path
  (model/attention/sparse.py:284-364, 420): layer 0, without a forecast, the
  static window; layers 1..11 per-query-block lists from the non-causal
  routing of the forecast layer L-1 emitted. Every layer's lists bit-exact
  against the oracle's, sampled attention rows of every layer within the bf16
  bar, finite logits.
* Offload at a 32K context (512 blocks of 64, model/attention/async_offload.py:
  170-519): the prefetch selection at lengths 32767 and 32768 in both routings
  (the 257-512-block selection tier), exact block fetches by both transfer
  methods, the offloaded decode step against the oracle, and the 12-layer
  async-prefetch model equal to the synchronous offload model over 3 steps
  with no stale prefetch; the same model replayed from a HIP graph with each
  prefetch carried by the previous layer's attention launch, every offloaded
  layer's selection and attention checked against the oracle at each step.
"""

import numpy as np
import pytest
import torch

import sparda
from sparda import synth
from model.attention import AsyncOffloadedKVCache, KVCache, OffloadedKVCache
from model.config import ModelConfig
from model.model import SparDAResearchModel
from oracle import sparda_oracle as O
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def test_twelve_layer_forward_at_16k_against_the_oracle(monkeypatch):
    case("12-layer forward T=16384 (chunked path)")
    T, bs, k = 16384, 64, 8
    cfg = ModelConfig(n_layer=12, context_length=T, block_size=bs, top_k_blocks=k,
                      attention_backend="hip_sparse", norm_eps=1e-5)
    torch.manual_seed(1003)
    model = SparDAResearchModel(cfg).to(DEV, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(1003)
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=g).to(DEV)
    prefills = []
    real_chunked = sparda.prefill_chunked

    def chunked_spy(q, kk, v, topk, block_size, top_k, **kw):
        # the same launch, with the lists it built written out for the check
        out, sel, n = real_chunked(q, kk, v, topk, block_size, top_k, want_sel=True)
        prefills.append({"q": q.detach().cpu(), "k": kk.detach().cpu(), "v": v.detach().cpu(),
                         "sel": sel.cpu().numpy(), "n": n.cpu().numpy(), "out": out.detach().cpu()})
        return out

    def per_token_spy(*a, **kw):
        raise AssertionError("a per-token prefill ran past 8192 tokens")

    monkeypatch.setattr(sparda, "prefill_chunked", chunked_spy)
    monkeypatch.setattr(sparda, "prefill_routed", per_token_spy)
    monkeypatch.setattr(sparda, "prefill", per_token_spy)
    with torch.no_grad():
        res = model(ids, return_forecasts=True)
    torch.cuda.synchronize()
    assert torch.isfinite(res["logits"]).all()
    assert len(prefills) == 12
    r = np.random.default_rng(16384)
    for L, p in enumerate(prefills):
        q, kk, v = np32(p["q"]), np32(p["k"]), np32(p["v"])
        tk = None
        if L > 0:
            # layer L routes with the forecast layer L-1 emitted, every row over all blocks
            _, tk, _, _ = O.route(np32(res["forecasts"][L - 1]), O.compress(kk, bs), bs, k, False)
        sel_o, n_o = O.chunked_selection(tk, 1, 4, T, bs, k)
        assert np.array_equal(p["n"], n_o) and np.array_equal(p["sel"], sel_o), f"layer {L}: selection"
        ts = sorted({int(t) for t in r.integers(0, T, 60)} | {0, 63, 64, T - 1})
        rows = [(0, t) for t in ts]
        want = O.attention_prefill(q, kk, v, sel_o, n_o, bs, True, rows=rows)
        got = np32(p["out"])
        assert_close_out(got[0, ts], want[0, ts], torch.bfloat16, what=f"layer {L} attention")


CTX = 32768


@pytest.fixture(scope="module")
def arena_32k():
    """One layer's KV at a 32K context in a pinned host arena (RoPE'd keys,
    N(0,1) values, bf16): the first 32767 tokens as one append, the last as a
    single-token append that continues the block sums; the copies the oracle
    reads."""
    B, Hkv, D, bs = 1, 4, 64, 64
    a = sparda.OffloadArena(B, CTX + 64, Hkv, D, torch.bfloat16, DEV)
    sums = torch.zeros(B, (CTX + 64) // bs, Hkv, D, dtype=torch.float32, device=DEV)
    ks, vs = [], []
    for p0, k, v in synth.kv_chunks(B, CTX, Hkv, D, seed=2001):
        ks.append(k.to(torch.bfloat16))
        vs.append(v.to(torch.bfloat16))
    K = torch.cat(ks, 1)
    V = torch.cat(vs, 1)
    a.append(K[:, :CTX - 1].to(DEV), V[:, :CTX - 1].to(DEV), 0, bs, sums)
    a.append(K[:, CTX - 1:].to(DEV), V[:, CTX - 1:].to(DEV), CTX - 1, bs, sums)
    torch.cuda.synchronize()
    assert np.array_equal((sums[:, :CTX // bs] / bs).cpu().numpy(), O.compress(np32(K), bs))
    yield {"arena": a, "sums": sums, "K": K, "V": V}
    a.close()


@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_prefetch_selection_and_fetch_at_512_blocks(arena_32k, routing):
    case(f"32K select + fetch {routing}")
    a, sums, K, V = arena_32k["arena"], arena_32k["sums"], arena_32k["K"], arena_32k["V"]
    B, Hkv, D, bs, k = 1, 4, 64, 64, 8
    g = torch.Generator().manual_seed(2002)
    f = torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16)
    kc = np.zeros((B, CTX + 64, Hkv, D), np.float32)
    kc[:, :CTX] = np32(K)
    for length in (CTX - 1, CTX):
        # the block sums of the first `length` tokens, recomputed from the arena
        sl = torch.full_like(sums, float("nan"))
        a.rebuild_sums(length, bs, sl)
        if length == CTX:
            assert torch.equal(sl[:, :CTX // bs], sums[:, :CTX // bs])
        sel, n = sparda.select_decode(f.to(DEV), sl, length, length, bs, k, routing=routing)
        torch.cuda.synchronize()
        sel_o, n_o = O.prefetch_selection(kc, length, length, np32(f), bs, k, routing)
        assert np.array_equal(n.cpu().numpy(), n_o) and np.array_equal(sel.cpu().numpy(), sel_o), length
        for method in (sparda.FETCH_KERNEL, sparda.FETCH_DMA):
            kb = torch.full((B, Hkv, k + 2, bs, D), 7.0, dtype=torch.bfloat16, device=DEV)
            vb = torch.full_like(kb, 7.0)
            a.fetch(sel, n, bs, length, kb, vb, method)
            torch.cuda.synchronize()
            kh, vh = kb.cpu(), vb.cpu()
            for h in range(Hkv):
                for i in range(int(n_o[0, h])):
                    j = int(sel_o[0, h, i])
                    rows = min(bs, length - j * bs)
                    assert torch.equal(kh[0, h, i, :rows], K[0, j * bs:j * bs + rows, h])
                    assert torch.equal(vh[0, h, i, :rows], V[0, j * bs:j * bs + rows, h])


def test_offloaded_decode_step_at_32k_against_the_oracle(arena_32k):
    case("32K offloaded decode step")
    a, K, V = arena_32k["arena"], arena_32k["K"], arena_32k["V"]
    B, Hq, Hkv, D, bs, k = 1, 12, 4, 64, 64, 8
    L = CTX - 1  # cached tokens when the prefetch is issued; the query is token L
    g = torch.Generator().manual_seed(2003)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    f = torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16)
    sums = torch.zeros(B, (CTX + 64) // bs, Hkv, D, dtype=torch.float32, device=DEV)
    a.rebuild_sums(L, bs, sums)
    sel, n = sparda.select_decode(f.to(DEV), sums, L, L, bs, k, routing="absolute")
    kb = torch.empty((B, Hkv, k + 2, bs, D), dtype=torch.bfloat16, device=DEV)
    vb = torch.empty_like(kb)
    a.fetch(sel, n, bs, L, kb, vb, sparda.FETCH_KERNEL)
    kn, vn = K[:, L].to(DEV), V[:, L].to(DEV)
    out = sparda.decode_selected(q.to(DEV), kb, vb, L + 1, bs, sel, n, compact=True, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    kc = np.zeros((B, CTX, Hkv, D), np.float32)
    kc[:, :CTX] = np32(K)
    vc = np32(V)
    sel_o, n_o = O.prefetch_selection(kc, L, L, np32(f), bs, k, "absolute")
    assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
    want = O.attention_decode(np32(q), kc, vc, L + 1, sel_o, n_o, bs)
    assert_close_out(np32(out), want, torch.bfloat16)


def test_twelve_layer_async_prefetch_model_at_32k_equals_sync_offload():
    case("12-layer async vs sync offload at 32K")
    bs, k, steps = 64, 8, 3
    cap = CTX + 64
    cfg = ModelConfig(n_layer=12, context_length=cap, block_size=bs, top_k_blocks=k, decode_routing="absolute",
                      attention_backend="async_offload", norm_eps=1e-5)
    torch.manual_seed(1004)
    ma = SparDAResearchModel(cfg).to(DEV, torch.bfloat16).eval()
    ms = SparDAResearchModel(ModelConfig(**{**cfg.__dict__, "attention_backend": "offload"})).to(
        DEV, torch.bfloat16).eval()
    ms.load_state_dict(ma.state_dict())
    ca = [KVCache(1, cap, 4, 64, DEV, torch.bfloat16)] + [
        AsyncOffloadedKVCache(1, cap, 4, 64, DEV, torch.bfloat16, block_size=bs) for _ in range(11)]
    cs = [KVCache(1, cap, 4, 64, DEV, torch.bfloat16)] + [
        OffloadedKVCache(1, cap, 4, 64, DEV, torch.bfloat16, block_size=bs) for _ in range(11)]
    for li in range(12):
        for _, kk, vv in synth.kv_chunks(1, CTX - 8, 4, 64, seed=2100 + li):
            kd, vd = kk.to(DEV, torch.bfloat16), vv.to(DEV, torch.bfloat16)
            ca[li].update(kd, vd)
            cs[li].update(kd, vd)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(1006)
    ids = torch.randint(0, cfg.vocab_size, (steps, 1, 1), generator=g).to(DEV)
    with torch.no_grad():
        for s in range(steps):
            la = ma(ids[s], kv_caches=ca)["logits"]
            ls = ms(ids[s], kv_caches=cs)["logits"]
            torch.cuda.synchronize()
            assert torch.isfinite(la).all()
            assert torch.equal(la, ls), f"step {s}: max diff {(la.float() - ls.float()).abs().max().item()}"
    assert all(c.current_len == CTX - 8 + steps for c in ca)
    assert sum(layer.attention.stale_prefetches for layer in ma.layers[1:]) == 0
    assert all(layer.attention.prefetched_bytes > 0 for layer in ma.layers[1:])


def test_twelve_layer_replayed_offload_steps_at_32k_against_the_oracle():
    # the 12-layer offloaded model at a 32K context decoded by GraphDecoder,
    # each layer's prefetch carried by the previous layer's attention launch:
    # at every replayed step, every offloaded layer's prefetched selection
    # (bit for bit) and attention output (bf16 bar) against the oracle, from
    # the q, routing forecast and output the replay left in its buffers and the
    # arena contents
    from model.decode_graph import GraphDecoder
    case("12-layer replayed offload steps at 32K vs the oracle (carried prefetch)")
    bs, k, steps = 64, 8, 2
    cap = CTX + 64
    cfg = ModelConfig(n_layer=12, context_length=cap, block_size=bs, top_k_blocks=k, decode_routing="absolute",
                      attention_backend="async_offload", norm_eps=1e-5)
    torch.manual_seed(1005)
    model = SparDAResearchModel(cfg).to(DEV, torch.bfloat16).eval()
    caches = [KVCache(1, cap, 4, 64, DEV, torch.bfloat16)] + [
        AsyncOffloadedKVCache(1, cap, 4, 64, DEV, torch.bfloat16, block_size=bs) for _ in range(11)]
    for li in range(12):
        for _, kk, vv in synth.kv_chunks(1, CTX - 8, 4, 64, seed=2200 + li):
            caches[li].update(kk.to(DEV, torch.bfloat16), vv.to(DEV, torch.bfloat16))
    torch.cuda.synchronize()
    gd = GraphDecoder(model, 1, cap, caches=caches, taps=tuple(range(1, 12)))
    assert gd.overlap == "fused"
    g = torch.Generator().manual_seed(1007)
    ids = torch.randint(0, cfg.vocab_size, (steps, 1, 1), generator=g).to(DEV)
    with torch.no_grad():
        for s in range(steps):
            logits = gd.step(ids[s])
            torch.cuda.synchronize()
            assert torch.isfinite(logits).all()
            S = gd.length
            for i in range(1, 12):
                case(f"  step {s}, position {S - 1}, layer {i}")
                c, tap = gd.caches[i], gd.tapped[i]
                kc, vc = c.cpu_k[:, :S].float().numpy(), c.cpu_v[:, :S].float().numpy()
                # the prefetch selected before the token at S - 1 was appended
                sel_o, n_o = O.prefetch_selection(kc, S - 1, S - 1, np32(tap["f"].reshape(1, 4, -1)), bs, k,
                                                  "absolute")
                assert np.array_equal(tap["n_sel"].cpu().numpy(), n_o)
                assert np.array_equal(tap["sel"].cpu().numpy(), sel_o)
                want = O.attention_decode(np32(tap["q"]), kc, vc, S, sel_o, n_o, bs)
                assert_close_out(np32(tap["out"]), want, torch.bfloat16, what=f"layer {i} at {S - 1}")
    assert gd.length == CTX - 8 + steps
