"""GPU parity of the selected-block decode and of the host-resident KV cache
(append, block sums, decode-time selection, block fetch) against the oracle.

Block sums / prototypes, selections and fetched bytes are compared exactly;
attention outputs within max-abs 2e-2 / mean-abs 2e-3 (bf16) or 1e-4 (fp32).
"""

import numpy as np
import pytest
import torch

import sparda
from sparda import synth
from oracle import sparda_oracle as O
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def _sums_as_protos(sums, length, bs):
    nb = (length + bs - 1) // bs
    return (sums[:, :nb] / bs).cpu().numpy()


# ---------------------------------------------------------------------------
# decode over a given selection
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_selected_in_place_matches_oracle_and_fused_decode(dtype):
    case(f"decode_selected in place {dtype}")
    B, S, Hq, Hkv, D, bs, k = 4, 5000, 12, 4, 64, 64, 8
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=dtype, seed=21)
    d = {n: t.to(DEV) for n, t in x.items()}
    out_f, ex = sparda.decode(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], bs, k, routing="absolute",
                              want_sel=True)
    out = sparda.decode_selected(d["q"], d["k_cache"], d["v_cache"], S, bs, ex["sel"], ex["n_sel"])
    torch.cuda.synchronize()
    kc, vc = np32(x["k_cache"]), np32(x["v_cache"])
    want = O.attention_decode(np32(x["q"]), kc, vc, S, ex["sel"].cpu().numpy(), ex["n_sel"].cpu().numpy(), bs)
    assert_close_out(np32(out), want, dtype)
    # the fused step runs the same attention kernel over the same blocks
    assert torch.equal(out, out_f)


@pytest.mark.parametrize("S", [1, 64, 65, 4097, 32768])
def test_decode_selected_dense_any_length(S):
    case(f"decode_selected dense S={S}")
    B, Hq, Hkv, D, bs = 1, 12, 4, 64, 64
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=torch.bfloat16, seed=22 + S)
    d = {n: t.to(DEV) for n, t in x.items()}
    out = sparda.decode_selected(d["q"], d["k_cache"], d["v_cache"], S, bs)
    torch.cuda.synchronize()
    NB = (S + bs - 1) // bs
    sel = np.arange(NB, dtype=np.int32).reshape(1, 1, NB).repeat(Hkv, axis=1).repeat(B, axis=0)
    n = np.full((B, Hkv), NB, np.int32)
    want = O.attention_decode(np32(x["q"]), np32(x["k_cache"]), np32(x["v_cache"]), S, sel, n, bs)
    assert_close_out(np32(out), want, torch.bfloat16)


@pytest.mark.parametrize("bs", [64, 32])
def test_dense_decode_split_over_workgroups(bs):
    """The dense decode split over workgroups (flash-decoding partials in a
    workspace, merged by a second launch) against the one-workgroup form
    through the C ABI and against the oracle; then decode_at at short
    positions of a long cache, where most splits hold no block."""
    from sparda._lib import call
    B, S, Hq, Hkv, D = 2, 9000, 12, 4, 64
    case(f"dense decode split bs={bs} B={B} S={S}")
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=torch.bfloat16, seed=24 + bs)
    d = {n: t.to(DEV) for n, t in x.items()}
    q, kc, vc = d["q"], d["k_cache"], d["v_cache"]
    nbytes = sparda.load().sparda_decode_dense_workspace_bytes(B, Hq, Hkv, D, S, bs)
    assert nbytes > 0
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=DEV)
    outs = {}
    for name, (wp, wb) in {"one": (None, 0), "split": (ws.data_ptr(), nbytes)}.items():
        o = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=DEV)
        kv_sb, kv_ss, kv_sh, _ = kc.stride()
        call("sparda_decode_selected", q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
                    kv_sb, kv_ss, kv_sh, 1, 0, None, None, 0, None, None, 0, 0, B, S, Hq, Hkv, D, bs,
                    D ** -0.5, o.data_ptr(), o.stride(0), wp, wb, torch.cuda.current_stream().cuda_stream)
        outs[name] = o
    torch.cuda.synchronize()
    NB = (S + bs - 1) // bs
    sel = np.arange(NB, dtype=np.int32).reshape(1, 1, NB).repeat(Hkv, axis=1).repeat(B, axis=0)
    n = np.full((B, Hkv), NB, np.int32)
    want = O.attention_decode(np32(x["q"]), np32(x["k_cache"]), np32(x["v_cache"]), S, sel, n, bs)
    for o in outs.values():
        assert_close_out(np32(o), want, torch.bfloat16)
    # the two forms differ only in the order partial sums are combined
    diff = (outs["one"].float() - outs["split"].float()).abs().max().item()
    assert diff <= 4e-3, diff
    # positions of a cache of 9000 rows: the split count follows max_len, the
    # blocks the position (splits past the last block hold none)
    for p in (0, 5, bs - 1, bs, 3 * bs + 7, 700, S - 1):
        case(f"dense decode_at split bs={bs} p={p}")
        pos = torch.tensor([p], dtype=torch.int64, device=DEV)
        o = sparda.decode_at(q, kc, vc, pos, bs, window=0)
        torch.cuda.synchronize()
        nb = p // bs + 1
        sel_p = np.arange(nb, dtype=np.int32).reshape(1, 1, nb).repeat(Hkv, axis=1).repeat(B, axis=0)
        want_p = O.attention_decode(np32(x["q"]), np32(x["k_cache"]), np32(x["v_cache"]), p + 1, sel_p,
                                    np.full((B, Hkv), nb, np.int32), bs)
        assert_close_out(np32(o), want_p, torch.bfloat16)


def test_decode_selected_new_token_override_and_invalid_slots():
    case("decode_selected k_new override, skipped blocks")
    B, S, Hq, Hkv, D, bs = 2, 700, 12, 4, 64, 64
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=torch.float32, seed=23)
    d = {n: t.to(DEV) for n, t in x.items()}
    kn, vn = d["k_cache"][:, S - 1].clone(), d["v_cache"][:, S - 1].clone()
    kc, vc = d["k_cache"].clone(), d["v_cache"].clone()
    kc[:, S - 1] = 7.0  # garbage where the new token lives: k_new/v_new must win
    vc[:, S - 1] = -7.0
    cb = (S - 1) // bs
    sel = torch.tensor([0, 3, cb, 99, -1], dtype=torch.int32).repeat(B, Hkv, 1).to(DEV)  # 99: beyond cb, skipped
    n = torch.full((B, Hkv), 5, dtype=torch.int32, device=DEV)
    out = sparda.decode_selected(d["q"], kc, vc, S, bs, sel, n, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    want_sel = np.array([0, 3, cb], np.int32).reshape(1, 1, 3).repeat(Hkv, 1).repeat(B, 0)
    want = O.attention_decode(np32(x["q"]), np32(x["k_cache"]), np32(x["v_cache"]), S, want_sel,
                              np.full((B, Hkv), 3), bs)
    assert_close_out(np32(out), want, torch.float32)


# ---------------------------------------------------------------------------
# host-resident KV arena
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def arena_bf16():
    a = sparda.OffloadArena(2, 4096, 4, 64, torch.bfloat16, DEV)
    yield a
    a.close()


def test_arena_views_are_pinned_and_zero(arena_bf16):
    case("arena views")
    a = arena_bf16
    assert a.k_host.shape == (2, 4096, 4, 64) and a.k_host.device.type == "cpu"
    assert a.k_host.is_pinned()


def test_arena_append_prefill_then_tokens_block_sums_exact(arena_bf16):
    case("arena append + block sums")
    a = arena_bf16
    B, Hkv, D, bs = 2, 4, 64, 64
    T = 1000
    g = torch.Generator().manual_seed(31)
    k = torch.randn(B, T + 200, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T + 200, Hkv, D, generator=g).to(torch.bfloat16)
    sums = torch.zeros(B, 4096 // bs, Hkv, D, dtype=torch.float32, device=DEV)
    kd, vd = k.to(DEV), v.to(DEV)
    a.append(kd[:, :T], vd[:, :T], 0, bs, sums)
    for t in range(T, T + 200):  # one token at a time across block boundaries
        a.append(kd[:, t:t + 1], vd[:, t:t + 1], t, bs, sums)
    torch.cuda.synchronize()
    L = T + 200
    assert torch.equal(a.k_host[:, :L], k) and torch.equal(a.v_host[:, :L], v)
    assert np.array_equal(_sums_as_protos(sums, L, bs), O.compress(np32(k), bs))
    # rebuilding from the arena (read through its device mapping) gives the same sums
    sums2 = torch.full_like(sums, float("nan"))
    a.rebuild_sums(L, bs, sums2)
    torch.cuda.synchronize()
    nb = (L + bs - 1) // bs
    assert torch.equal(sums2[:, :nb], sums[:, :nb])


def test_arena_append_strided_source_fp32():
    case("arena append strided fp32")
    a = sparda.OffloadArena(1, 256, 2, 32, torch.float32, DEV)
    try:
        g = torch.Generator().manual_seed(32)
        big = torch.randn(1, 100, 3, 32, generator=g)  # head 1 and 2 of 3: strided view
        k = big[:, :, 1:].to(DEV)
        v = (big[:, :, 1:] * 2).to(DEV)
        sums = torch.zeros(1, 16, 2, 32, device=DEV)
        a.append(k, v, 0, 16, sums)
        torch.cuda.synchronize()
        assert torch.equal(a.k_host[:, :100], big[:, :, 1:]) and torch.equal(a.v_host[:, :100], big[:, :, 1:] * 2)
        assert np.array_equal(_sums_as_protos(sums, 100, 16), O.compress(big[:, :, 1:].numpy(), 16))
    finally:
        a.close()


@pytest.mark.parametrize("length", [20, 640, 1000, 1024, 4095])
@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_select_decode_matches_oracle(arena_bf16, length, routing):
    case(f"select_decode len={length} {routing}")
    a = arena_bf16
    B, Hkv, D, bs, k = 2, 4, 64, 64, 8
    g = torch.Generator().manual_seed(40 + length)
    kk = torch.randn(B, length, Hkv, D, generator=g).to(torch.bfloat16)
    f = torch.randn(B, Hkv, D, generator=g).to(torch.bfloat16)
    sums = torch.zeros(B, 4096 // bs, Hkv, D, dtype=torch.float32, device=DEV)
    a.append(kk.to(DEV), kk.to(DEV), 0, bs, sums)
    sel, n = sparda.select_decode(f.to(DEV), sums, length, length, bs, k, routing=routing)
    torch.cuda.synchronize()
    kc = np.zeros((B, 4096, Hkv, D), np.float32)
    kc[:, :length] = np32(kk)
    sel_o, n_o = O.prefetch_selection(kc, length, length, np32(f), bs, k, routing)
    assert np.array_equal(n.cpu().numpy(), n_o)
    assert np.array_equal(sel.cpu().numpy(), sel_o)


@pytest.mark.parametrize("method", [sparda.FETCH_KERNEL, sparda.FETCH_DMA])
def test_fetch_blocks_exact(arena_bf16, method):
    case(f"fetch method={method}")
    a = arena_bf16
    B, Hkv, D, bs = 2, 4, 64, 64
    L = 1000
    g = torch.Generator().manual_seed(50)
    k = torch.randn(B, L, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, L, Hkv, D, generator=g).to(torch.bfloat16)
    a.append(k.to(DEV), v.to(DEV), 0)
    cap = 10
    rng = np.random.default_rng(51)
    sel = np.full((B, Hkv, cap), -1, np.int32)
    n = np.zeros((B, Hkv), np.int32)
    for b in range(B):
        for h in range(Hkv):
            m = int(rng.integers(1, cap + 1))
            blocks = np.sort(rng.choice(16, size=m, replace=False)).astype(np.int32)  # 16 blocks incl. partial 15
            sel[b, h, :m] = blocks
            n[b, h] = m
    kd = torch.full((B, Hkv, cap, bs, D), 3.0, dtype=torch.bfloat16, device=DEV)
    vd = torch.full_like(kd, 3.0)
    a.fetch(torch.from_numpy(sel).to(DEV), torch.from_numpy(n).to(DEV), bs, L, kd, vd, method)
    torch.cuda.synchronize()
    kh, vh = kd.cpu(), vd.cpu()
    for b in range(B):
        for h in range(Hkv):
            for i in range(cap):
                if i < n[b, h]:
                    j = int(sel[b, h, i])
                    rows = min(bs, L - j * bs)
                    assert torch.equal(kh[b, h, i, :rows], k[b, j * bs:j * bs + rows, h])
                    assert torch.equal(vh[b, h, i, :rows], v[b, j * bs:j * bs + rows, h])
                    assert (kh[b, h, i, rows:] == 3.0).all()  # rows >= length untouched
                else:
                    assert (kh[b, h, i] == 3.0).all()  # unused slots untouched


@pytest.mark.parametrize("method,bs,k", [(sparda.FETCH_KERNEL, 64, 8), (sparda.FETCH_DMA, 64, 8),
                                         (sparda.FETCH_KERNEL, 32, 4)])
def test_offload_decode_step_equals_resident_attention(method, bs, k):
    # the prefetched (compact) blocks + the new token attended = the same
    # selection attended in place on a GPU-resident cache
    case(f"offload decode step method={method} bs={bs}")
    B, S, Hq, Hkv, D = 1, 8000, 12, 4, 64
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=torch.bfloat16, seed=60, capacity=8192)
    d = {n_: t.to(DEV) for n_, t in x.items()}
    L = S - 1  # tokens in the cache when the prefetch is issued
    a = sparda.OffloadArena(B, 8192, Hkv, D, torch.bfloat16, DEV)
    try:
        sums = torch.zeros(B, 8192 // bs, Hkv, D, dtype=torch.float32, device=DEV)
        a.append(d["k_cache"][:, :L], d["v_cache"][:, :L], 0, bs, sums)
        sel, n = sparda.select_decode(d["forecast"], sums, L, L, bs, k, routing="absolute")
        kb = torch.empty((B, Hkv, k + 2, bs, D), dtype=torch.bfloat16, device=DEV)
        vb = torch.empty_like(kb)
        a.fetch(sel, n, bs, L, kb, vb, method)
        kn, vn = d["k_cache"][:, L], d["v_cache"][:, L]
        out = sparda.decode_selected(d["q"], kb, vb, S, bs, sel, n, compact=True, k_new=kn, v_new=vn)
        ref = sparda.decode_selected(d["q"], d["k_cache"], d["v_cache"], S, bs, sel, n)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        kc = np32(x["k_cache"])
        sel_o, n_o = O.prefetch_selection(kc, L, L, np32(x["forecast"]), bs, k, "absolute")
        assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
        want = O.attention_decode(np32(x["q"]), kc, np32(x["v_cache"]), S, sel_o, n_o, bs)
        assert_close_out(np32(out), want, torch.bfloat16)
    finally:
        a.close()
