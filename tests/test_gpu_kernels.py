"""GPU parity of libsparda's kernels against the CPU oracle.

Integer/index outputs (prototypes, scores, top-k, selection lists) are
compared bit-exactly; attention outputs within max-abs 2e-2 / mean-abs 2e-3
(bf16) or max-abs 1e-4 (fp32).
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


# ---------------------------------------------------------------------------
# compressor
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,S,H,D,bs,dtype", [
    (4, 4096, 4, 64, 64, torch.bfloat16),   # prefill workload (B=4, T=4096)
    (1, 1024, 4, 64, 64, torch.float32),    # fp32 layer at T=1024
    (2, 50, 4, 32, 16, torch.float32),      # tests/test_forecast.py:64-68 padding case
    (3, 1000, 2, 16, 48, torch.bfloat16),   # ragged tail, odd block size
    (8, 16384, 4, 64, 64, torch.bfloat16),  # decode cache at 16K
])
def test_compress_bit_exact(B, S, H, D, bs, dtype):
    case(f"compress B={B} S={S} H={H} D={D} bs={bs} {dtype}")
    k = torch.randn(B, S, H, D, generator=torch.Generator().manual_seed(S)).to(dtype)
    got = sparda.compress(k.to(DEV), bs).cpu().numpy()
    want = O.compress(np32(k), bs)
    assert got.shape == want.shape
    assert np.array_equal(got, want)


def test_compress_strided_view():
    case("compress strided view")
    big = torch.randn(2, 300, 6, 64, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    view = big[:, :, 1:5, :]  # stride_h = 64, stride_s = 384
    got = sparda.compress(big.to(DEV)[:, :, 1:5, :], 64).cpu().numpy()
    assert np.array_equal(got, O.compress(np32(view), 64))


# ---------------------------------------------------------------------------
# router
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,Tq,H,Df,bs,k,fdtype,causal,pos0", [
    (1, 1024, 4, 64, 64, 8, torch.float32, True, 0),     # fp32 layer at T=1024 (NB=16)
    (4, 4096, 4, 64, 64, 8, torch.bfloat16, True, 0),    # prefill workload (NB=64)
    (2, 333, 2, 32, 16, 2, torch.float32, True, 0),      # reference test geometry, ragged
    (2, 256, 4, 64, 64, 8, torch.bfloat16, False, 0),    # non-causal selector
    (1, 3, 4, 64, 64, 8, torch.float32, True, 16383),    # decode rows at the end of a 16K cache
    (1, 2048, 2, 128, 32, 16, torch.bfloat16, True, 0),  # k=16, Df=128
    (1, 512, 2, 16, 8, 32, torch.float32, True, 0),      # k=32, many blocks
])
def test_route_bit_exact(B, Tq, H, Df, bs, k, fdtype, causal, pos0):
    case(f"route B={B} Tq={Tq} H={H} Df={Df} bs={bs} k={k} {fdtype} causal={causal} pos0={pos0}")
    g = torch.Generator().manual_seed(Tq + k)
    S = max(Tq, pos0 + Tq)
    kk = torch.randn(B, S, H, Df, generator=g)
    f = torch.randn(B, Tq, H, Df, generator=g).to(fdtype)
    P = O.compress(kk.numpy(), bs)
    topk, scores, sel, n = sparda.route(f.to(DEV), torch.from_numpy(P).to(DEV), bs, k, causal=causal,
                                        score_pos0=pos0, query_pos0=pos0, want_topk=True, want_scores=True,
                                        want_sel=True)
    sc_o, tk_o, sel_o, n_o = O.route(np32(f), P, bs, k, causal, pos0, pos0)
    assert np.array_equal(scores.cpu().numpy(), sc_o)
    assert np.array_equal(topk.cpu().numpy(), tk_o)
    assert np.array_equal(n.cpu().numpy(), n_o)
    assert np.array_equal(sel.cpu().numpy(), sel_o)


def test_route_ties_and_reference_decode_row():
    case("route ties")
    # all-equal prototypes -> every score ties; lower index must win
    B, Tq, H, D, bs, k = 1, 700, 2, 64, 64, 8
    P = np.ones((B, 11, H, D), np.float32)
    f = torch.ones(B, Tq, H, D)
    topk, _, sel, n = sparda.route(f.to(DEV), torch.from_numpy(P).to(DEV), bs, k, want_sel=True)
    _, tk_o, sel_o, n_o = O.route(f.numpy(), P, bs, k)
    assert np.array_equal(topk.cpu().numpy(), tk_o)
    assert np.array_equal(sel.cpu().numpy(), sel_o)
    assert topk[0, 0, 699].tolist() == list(range(8))


def test_topk_identical_scores_both_algorithms():
    case("topk on identical scores")
    r = np.random.default_rng(3)
    s = r.integers(-4, 4, size=(300, 256)).astype(np.float32)
    s[r.random(s.shape) < 0.3] = -np.inf
    s[:, 7] = -0.0
    want = O.topk(s, 8)
    for algo in (sparda.TOPK_ROWS, sparda.TOPK_WAVE):
        got = sparda.topk_scores(torch.from_numpy(s).to(DEV), 8, algo).cpu().numpy()
        assert np.array_equal(got, want), f"algo {algo}"


def test_topk_on_reference_path_scores():
    """Scores produced by the op-for-op reference restatement (torch matmul +
    masked_fill) are fed unchanged to the GPU selection stage."""
    case("topk on reference-path scores")
    from oracle import reference_path as R
    g = torch.Generator().manual_seed(5)
    k = torch.randn(2, 4096, 4, 64, generator=g)
    f = torch.randn(2, 4096, 4, 64, generator=g)
    sc, tk_ref = R.select_blocks(f, R.block_means(k, 64), 64, 8)
    sc = sc.contiguous()
    want = O.topk(sc.numpy(), 8)
    for algo in (sparda.TOPK_ROWS, sparda.TOPK_WAVE):
        got = sparda.topk_scores(sc.to(DEV), 8, algo).cpu().numpy()
        assert np.array_equal(got, want)
    # where no tie is involved (at least k finite scores), torch.topk agrees too
    fin = np.isfinite(sc.numpy()).sum(-1) >= 8
    assert np.array_equal(want[fin], tk_ref.numpy()[fin])


@pytest.mark.parametrize("mode,Tq,NB,bs,k,pos0", [
    (sparda.SEL_DENSE, 1, 9, 64, 8, 520),
    (sparda.SEL_WINDOW_DECODE, 1, 256, 64, 8, 16383),
    (sparda.SEL_WINDOW_DECODE, 1, 256, 64, 8, 200),
    (sparda.SEL_WINDOW_PREFILL, 1000, 16, 64, 8, 0),
])
def test_select_fixed(mode, Tq, NB, bs, k, pos0):
    case(f"select_fixed mode={mode}")
    cap = NB if mode == sparda.SEL_DENSE else k + 2
    sel, n = sparda.select_fixed(mode, 2, Tq, 3, NB, bs, k, pos0, device=DEV, sel_cap=cap)
    sel_o, n_o = O.sel_fixed(mode, 2, Tq, 3, NB, bs, k, pos0, cap=cap)
    assert np.array_equal(n.cpu().numpy(), n_o)
    assert np.array_equal(sel.cpu().numpy(), sel_o)


def test_gather_reference_known_answer():
    # tests/test_sparse_attention.py:33-60
    case("gather")
    g = torch.Generator().manual_seed(0)
    k = torch.randn(2, 2, 48, 32, generator=g)
    v = torch.randn(2, 2, 48, 32, generator=g)
    idx = torch.tensor([[[0, 2], [1, 2]], [[2, 0], [0, 1]]])
    kg, vg = sparda.gather_blocks(k.to(DEV), v.to(DEV), idx.to(DEV), 16)
    assert kg.shape == (2, 2, 32, 32)
    assert torch.equal(kg[0, 0, :16].cpu(), k[0, 0, :16])
    assert torch.equal(kg[0, 0, 16:].cpu(), k[0, 0, 32:48])
    ko, vo = O.gather_blocks(k.numpy(), v.numpy(), idx.numpy(), 16)
    assert np.array_equal(kg.cpu().numpy(), ko) and np.array_equal(vg.cpu().numpy(), vo)
    kb, _ = sparda.gather_blocks(k[:, :, :40].to(DEV).to(torch.bfloat16), v[:, :, :40].to(DEV).to(torch.bfloat16),
                                 idx.to(DEV), 16)
    assert not kb[0, 0, 24:].float().any()


# ---------------------------------------------------------------------------
# prefill attention
# ---------------------------------------------------------------------------

def _prefill_case(B, T, Hq, Hkv, D, bs, k, dtype, seed, causal=True, dense=False, rows=None):
    x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=dtype, seed=seed)
    d = {n: t.to(DEV) for n, t in x.items()}
    if dense:
        sel = n = None
        sel_o = n_o = None
    else:
        protos = sparda.compress(d["k"], bs)
        _, _, sel, n = sparda.route(d["forecast"], protos, bs, k, causal=causal, want_topk=False, want_sel=True)
        _, _, sel_o, n_o = O.route(np32(x["forecast"]), O.compress(np32(x["k"]), bs), bs, k, causal)
        assert np.array_equal(sel.cpu().numpy(), sel_o)
    out = sparda.prefill(d["q"], d["k"], d["v"], sel, n, bs, causal=causal)
    torch.cuda.synchronize()
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, bs, causal, rows=rows)
    got = np32(out)
    mask = None
    if rows is not None:
        mask = np.zeros(got.shape, bool)
        for b, t in rows:
            mask[b, t] = True
    return assert_close_out(got, want, dtype, mask)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefill_layer_t1024(dtype):
    # single layer, B=1, T=1024, 12/4 heads, D=64, bs=64 (NB=16), k=8
    case(f"prefill T=1024 {dtype}")
    _prefill_case(1, 1024, 12, 4, 64, 64, 8, dtype, seed=1000)


@pytest.mark.parametrize("R", [1, 2, 3, 4])
def test_prefill_mfma_group_sizes_ragged(R):
    case(f"prefill mfma R={R} T=1000")
    _prefill_case(2, 1000, 4 * R, 4, 64, 64, 8, torch.bfloat16, seed=50 + R)


def test_prefill_mfma_dense_and_noncausal():
    case("prefill mfma dense + noncausal")
    _prefill_case(1, 700, 12, 4, 64, 64, 8, torch.bfloat16, seed=61, dense=True)
    _prefill_case(1, 700, 12, 4, 64, 64, 8, torch.bfloat16, seed=62, causal=False)
    _prefill_case(1, 300, 12, 4, 64, 64, 8, torch.bfloat16, seed=63, causal=False, dense=True)


@pytest.mark.parametrize("R", [1, 2, 3, 4])
def test_prefill_dense_kernel_group_sizes_and_ragged_lengths(R):
    # steps without lists (the reference's dense fallback, sparse.py:201-224):
    # 128-token windows, ragged last windows and blocks, causal and not
    for B, T, causal in ((2, 1000, True), (1, 129, True), (1, 1, True), (1, 65, False), (1, 200, False),
                         (1, 256, True)):
        case(f"prefill dense R={R} B={B} T={T} causal={causal}")
        _prefill_case(B, T, 4 * R, 4, 64, 64, 8, torch.bfloat16, seed=90 + R + T, causal=causal, dense=True)


def test_prefill_dense_kernel_16k_sampled_rows():
    # the dense causal layer of the 12-layer forward's shape (B=1, T=16384)
    case("prefill dense B=1 T=16384")
    r = np.random.default_rng(12)
    rows = sorted({(0, int(t)) for t in r.integers(0, 16384, 48)} | {(0, 0), (0, 127), (0, 128), (0, 16383)})
    _prefill_case(1, 16384, 12, 4, 64, 64, 8, torch.bfloat16, seed=1003, dense=True, rows=rows)


def test_prefill_general_kernel_shapes():
    # reference test geometry: 8 q heads / 2 kv heads, D=32, bs=16, k=2
    case("prefill general D=32 bs=16")
    _prefill_case(2, 64, 8, 2, 32, 16, 2, torch.float32, seed=70)
    _prefill_case(1, 333, 8, 2, 32, 16, 2, torch.bfloat16, seed=71)
    _prefill_case(1, 200, 4, 1, 128, 32, 3, torch.float32, seed=72)


def test_prefill_full_size_sampled_rows():
    # prefill workload: B=4, T=4096, 12/4 heads, D=64, bs=64 (NB=64), k=8, bf16
    case("prefill B=4 T=4096 sampled")
    r = np.random.default_rng(0)
    rows = sorted({(int(b), int(t)) for b, t in zip(r.integers(0, 4, 384), r.integers(0, 4096, 384))})
    rows += [(b, t) for b in range(4) for t in (0, 63, 64, 4095)]
    _prefill_case(4, 4096, 12, 4, 64, 64, 8, torch.bfloat16, seed=1001, rows=rows)


def test_prefill_long_context_16k_sampled_rows_and_selection_invariants():
    # T = 16384 (256 blocks): the per-token rule at a length where the backend
    # takes the chunked path by default (the kernels serve both; a caller keeps
    # this rule with use_chunked_gather=False), checked against the oracle on
    # sampled rows, plus the invariants of every selection list
    case("prefill B=1 T=16384 sampled")
    T, bs, k = 16384, 64, 8
    r = np.random.default_rng(5)
    rows = sorted({(0, int(t)) for t in r.integers(0, T, 160)} | {(0, t) for t in (0, 63, 64, 8191, 8192, T - 1)})
    _prefill_case(1, T, 12, 4, 64, bs, k, torch.bfloat16, seed=1005, rows=rows)
    x = synth.prefill_inputs(1, T, 12, 4, 64, dtype=torch.bfloat16, seed=1005)
    d = {n: t.to(DEV) for n, t in x.items()}
    _, _, sel, n = sparda.route(d["forecast"], sparda.compress(d["k"], bs), bs, k, want_topk=False, want_sel=True)
    sel, n = sel.cpu().numpy(), n.cpu().numpy()
    own = np.arange(T) // bs
    assert (n >= 1).all() and (n <= k + 2).all()
    assert (sel[..., 0] == 0).all()                                        # sink first
    last = np.take_along_axis(sel, (n - 1)[..., None].astype(np.int64), -1)[..., 0]
    assert (last == own[None, None, :]).all()                              # own block last
    valid = np.arange(sel.shape[-1])[None, None, None, :] < n[..., None]
    assert (np.where(valid, sel, 0) <= own[None, None, :, None]).all()     # causal
    d_sel = np.diff(np.where(valid, sel, 1 << 30), axis=-1)
    assert (d_sel[valid[..., 1:]] > 0).all()                               # ascending, no duplicates
    assert (n[..., own >= k - 1] >= k).all()                               # k distinct picks once k blocks exist


def test_prefill_at_the_largest_block_count_sampled_rows():
    # T = 65536: 1024 blocks, the most the matrix-core prefill's per-token
    # selection bitmasks hold; sampled rows against the oracle
    case("prefill B=1 T=65536 sampled")
    T, bs, k = 65536, 64, 8
    r = np.random.default_rng(9)
    ts = sorted({int(t) for t in r.integers(0, T, 96)} | {0, 63, 64, 32768, T - 64, T - 1})
    x = synth.prefill_inputs(1, T, 12, 4, 64, dtype=torch.bfloat16, seed=1009)
    d = {n: t.to(DEV) for n, t in x.items()}
    _, _, sel, n = sparda.route(d["forecast"], sparda.compress(d["k"], bs), bs, k, want_topk=False, want_sel=True)
    out = sparda.prefill(d["q"], d["k"], d["v"], sel, n, bs)
    torch.cuda.synchronize()
    sel, n = sel.cpu().numpy(), n.cpu().numpy()
    protos = O.compress(np32(x["k"]), bs)
    f = np32(x["forecast"])
    for t in ts:  # the oracle's selection of row t alone (its position passed explicitly)
        _, _, s_o, n_o = O.route(f[:, t:t + 1], protos, bs, k, True, score_pos0=t, query_pos0=t)
        assert np.array_equal(n[:, :, t], n_o[:, :, 0]) and np.array_equal(sel[:, :, t], s_o[:, :, 0]), f"row {t}"
    rows = [(0, t) for t in ts]
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel, n, bs, True, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(out), want, torch.bfloat16, mask)


def test_prefill_topk_covering_all_blocks_equals_dense():
    # k >= NB selects every causal block: the compacted per-token kernel and the
    # dense kernel (no lists) compute the same attention
    case("prefill k>=NB == dense")
    x = synth.prefill_inputs(1, 640, 12, 4, 64, dtype=torch.bfloat16, seed=80)
    d = {n: t.to(DEV) for n, t in x.items()}
    protos = sparda.compress(d["k"], 64)
    _, _, sel, n = sparda.route(d["forecast"], protos, 64, 10, want_topk=False, want_sel=True)
    a = sparda.prefill(d["q"], d["k"], d["v"], sel, n, 64)
    b = sparda.prefill(d["q"], d["k"], d["v"], None, None, 64)
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), None, None, 64, True)
    assert_close_out(np32(a), want, torch.bfloat16)
    assert_close_out(np32(b), want, torch.bfloat16)
    assert (a.float() - b.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("bs", [64, 32])
def test_prefill_is_deterministic(bs):
    # columns receive their blocks' contributions in block order whatever the
    # timing of the wavefronts: repeated launches agree bit for bit
    case(f"prefill repeat B=4 T=4096 bs={bs}")
    x = synth.prefill_inputs(4, 4096, 12, 4, 64, dtype=torch.bfloat16, seed=1001)
    d = {n: t.to(DEV) for n, t in x.items()}
    k = 8 if bs == 64 else 4
    _, _, sel, n = sparda.route(d["forecast"], sparda.compress(d["k"], bs), bs, k, want_topk=False, want_sel=True)
    a = sparda.prefill(d["q"], d["k"], d["v"], sel, n, bs)
    for _ in range(3):
        assert torch.equal(sparda.prefill(d["q"], d["k"], d["v"], sel, n, bs), a)


@pytest.mark.parametrize("bs,k", [(64, 8), (32, 4)])
def test_prefill_tiny_and_edge_lengths(bs, k):
    # lengths around one and two blocks and single tokens: the dense fallback
    # (at most two blocks), the first routed lengths, ragged last blocks
    for T in (1, 2, bs - 1, bs, bs + 1, 2 * bs + 1, 3 * bs, 5 * bs - 1):
        case(f"prefill T={T} bs={bs}")
        _prefill_case(2, T, 12, 4, 64, bs, k, torch.bfloat16, seed=300 + T)


@pytest.mark.parametrize("R", [1, 3, 4])
def test_prefill_block32_reference_default_config(R):
    # the reference's default configuration (configs/base.yaml:19-20): blocks of
    # 32 keys, top-4, on the matrix-core kernel; ragged T, causal and not
    case(f"prefill bs=32 k=4 R={R} T=1000")
    _prefill_case(2, 1000, 4 * R, 4, 64, 32, 4, torch.bfloat16, seed=80 + R)
    _prefill_case(1, 777, 4 * R, 4, 64, 32, 4, torch.bfloat16, seed=90 + R, causal=False)


def test_prefill_block32_full_size_sampled_rows_and_dense():
    # B=4, T=4096 with 32-key blocks (128 blocks), top-4 and top-8, sampled rows;
    # the dense step (no lists) with bs=32 equals the dense oracle
    case("prefill B=4 T=4096 bs=32 sampled")
    r = np.random.default_rng(3)
    rows = sorted({(int(b), int(t)) for b, t in zip(r.integers(0, 4, 256), r.integers(0, 4096, 256))})
    rows += [(b, t) for b in range(4) for t in (0, 31, 32, 63, 64, 4095)]
    _prefill_case(4, 4096, 12, 4, 64, 32, 4, torch.bfloat16, seed=1001, rows=rows)
    _prefill_case(4, 4096, 12, 4, 64, 32, 8, torch.bfloat16, seed=1001, rows=rows)
    _prefill_case(1, 700, 12, 4, 64, 32, 4, torch.bfloat16, seed=64, dense=True)


def _lists(rows, B, Hkv, T, cap):
    sel = np.full((B, Hkv, T, cap), -1, np.int32)
    n = np.zeros((B, Hkv, T), np.int32)
    for (b, g, t), lst in rows.items():
        sel[b, g, t, :len(lst)] = lst
        n[b, g, t] = len(lst)
    return sel, n


def _clean(sel, n, T, bs, causal):
    # set semantics of the kernel's contract: blocks outside [0, NB) (or past the
    # query's own block when causal) attend nothing, repeats count once
    NB = (T + bs - 1) // bs
    out = np.full_like(sel, -1)
    no = np.zeros_like(n)
    B, H, TT, cap = sel.shape
    for b in range(B):
        for g in range(H):
            for t in range(TT):
                top = t // bs if causal else NB - 1
                keep = sorted({int(j) for j in sel[b, g, t, :n[b, g, t]] if 0 <= j <= top})
                out[b, g, t, :len(keep)] = keep
                no[b, g, t] = len(keep)
    return out, no


@pytest.mark.parametrize("bs", [64, 32])
def test_prefill_irregular_selection_lists(bs):
    # unsorted lists, repeats, negative and future entries, lists without the sink
    # or the own block (the reference maximum then comes from another allowed key);
    # with 32-key blocks a future block can lie inside the token's 64-token window
    case(f"prefill irregular lists T=640 bs={bs}")
    B, T, Hq, Hkv, cap = 1, 640, 12, 4, 10
    x = synth.prefill_inputs(B, T, Hq, Hkv, 64, dtype=torch.bfloat16, seed=91)
    rng = np.random.default_rng(91)
    rows = {}
    for g in range(Hkv):
        for t in range(T):
            own = t // bs
            lst = list(rng.choice(own + 1, size=min(own + 1, int(rng.integers(1, 6))), replace=False))
            r = rng.random()
            if r < 0.2:
                lst = lst + [lst[0]]                  # repeat
            elif r < 0.3:
                lst = [-1] + lst                      # negative entry
            elif r < 0.4 and own + 1 < T // bs:
                lst = lst + [own + 1]                 # a future block
            rows[(0, g, t)] = [int(j) for j in lst][:cap]
    sel, n = _lists(rows, B, Hkv, T, cap)
    d = {k_: t_.to(DEV) for k_, t_ in x.items()}
    out = sparda.prefill(d["q"], d["k"], d["v"], torch.from_numpy(sel).to(DEV), torch.from_numpy(n).to(DEV), bs)
    cs, cn = _clean(sel, n, T, bs, True)
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), cs, cn, bs, True)
    assert_close_out(np32(out), want, torch.bfloat16)


def test_prefill_scores_far_above_the_reference_maximum():
    # a key scoring ~150 log2-units above both the sink and the diagonal key
    # trips the row-sum guard: the window is redone with its exact row maxima
    case("prefill exact-max fallback")
    B, T, Hq, Hkv, bs = 1, 256, 3, 1, 64
    x = synth.prefill_inputs(B, T, Hq, Hkv, 64, dtype=torch.float32, seed=93)
    q, k, v = x["q"].clone(), x["k"].clone(), x["v"].clone()
    e1 = torch.zeros(64)
    e1[0] = 20.0
    t_hot, s_hot = 200, 70      # token 200 (block 3) and a key of block 1
    q[0, t_hot, :, :] = e1
    k[0, t_hot, 0] = -e1        # its own key
    k[0, 0, 0] = -e1            # the sink key
    k[0, s_hot, 0] = e1         # dot = 400 -> 50 natural units above 0, 100 above the references
    q, k, v = (t_.to(torch.bfloat16) for t_ in (q, k, v))
    rows = {(0, 0, t): sorted({0, t // bs} | ({1} if t // bs >= 1 else set())) for t in range(T)}
    sel, n = _lists(rows, B, Hkv, T, 4)
    out = sparda.prefill(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(sel).to(DEV),
                         torch.from_numpy(n).to(DEV), bs)
    want = O.attention_prefill(np32(q), np32(k), np32(v), sel, n, bs, True)
    assert_close_out(np32(out), want, torch.bfloat16)
    # the hot row is (almost) exactly v[s_hot]
    hot = np32(out)[0, t_hot].reshape(Hq, 64)
    assert np.abs(hot - np32(v)[0, s_hot, 0][None, :]).max() <= 2e-2


@pytest.mark.parametrize("hot", [True, False])
def test_prefill_dense_kernel_scores_far_above_block_zero(hot):
    # the dense kernel's references are block 0's column maxima; a key ~72
    # log2-units above them trips the row-sum guard and the window is walked
    # again for the exact maxima (hot); 40 log2-units above stays on the
    # first walk (P up to 2^40, not hot)
    case(f"prefill dense, a key far above block 0 (hot={hot})")
    B, T, Hq, Hkv, bs = 1, 256, 12, 4, 64
    x = synth.prefill_inputs(B, T, Hq, Hkv, 64, dtype=torch.float32, seed=94)
    q, k, v = x["q"].clone(), x["k"].clone(), x["v"].clone()
    e1 = torch.zeros(64)
    e1[0] = 20.0 if hot else 15.0
    t_hot, s_hot = 200, 70      # token 200 (block 3) and a key of block 1
    q[0, t_hot, :, :] = e1
    k[0, t_hot, :] = -e1
    k[0, 0, :] = -e1
    k[0, s_hot, :] = e1         # dot 400 (225): 72 (40) log2-units above 0
    q, k, v = (t_.to(torch.bfloat16) for t_ in (q, k, v))
    out = sparda.prefill(q.to(DEV), k.to(DEV), v.to(DEV), None, None, bs)
    want = O.attention_prefill(np32(q), np32(k), np32(v), None, None, bs, True)
    assert_close_out(np32(out), want, torch.bfloat16)
    hot_row = np32(out)[0, t_hot].reshape(Hq, 64)
    assert np.abs(hot_row - np32(v)[0, s_hot].repeat(Hq // Hkv, axis=0)).max() <= 2e-2


# ---------------------------------------------------------------------------
# routed prefill (router folded into the attention launch)
# ---------------------------------------------------------------------------

def _routed_case(B, T, Hq, Hkv, D, bs, k, seed, causal=True, fdtype=None, dtype=torch.bfloat16):
    """prefill_routed against route + prefill on the same inputs: the lists
    and the attention output equal bit for bit, with and without the lists
    written out."""
    x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=dtype, seed=seed)
    d = {n: t.to(DEV) for n, t in x.items()}
    f = d["forecast"] if fdtype is None else d["forecast"].to(fdtype)
    protos = sparda.compress(d["k"], bs)
    _, _, sel, n = sparda.route(f, protos, bs, k, causal=causal, want_topk=False, want_sel=True)
    want = sparda.prefill(d["q"], d["k"], d["v"], sel, n, bs, causal=causal)
    got, sel2, n2 = sparda.prefill_routed(d["q"], d["k"], d["v"], f, protos, bs, k, causal=causal, want_sel=True)
    got_plain = sparda.prefill_routed(d["q"], d["k"], d["v"], f, protos, bs, k, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(n2, n) and torch.equal(sel2, sel), "routed lists differ from the router's"
    assert torch.equal(got, want), f"max diff {(got.float() - want.float()).abs().max().item()}"
    assert torch.equal(got_plain, want)
    return x, sel, n, got


@pytest.mark.parametrize("R", [1, 2, 3, 4])
@pytest.mark.parametrize("bs,k", [(64, 8), (32, 4)])
def test_prefill_routed_equals_route_then_prefill(R, bs, k):
    case(f"prefill_routed R={R} bs={bs} k={k} T=1000")
    _routed_case(2, 1000, 4 * R, 4, 64, bs, k, seed=400 + R)
    _routed_case(1, 777, 4 * R, 4, 64, bs, k, seed=410 + R, causal=False)


def test_prefill_routed_full_size_against_the_oracle():
    # prefill workload: B=4, T=4096, 12/4 heads, bs 64, top-8; lists against the
    # oracle's router, sampled rows against the oracle's attention
    case("prefill_routed B=4 T=4096")
    x, sel, n, got = _routed_case(4, 4096, 12, 4, 64, 64, 8, seed=1001)
    _, _, sel_o, n_o = O.route(np32(x["forecast"]), O.compress(np32(x["k"]), 64), 64, 8, True)
    assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
    r = np.random.default_rng(11)
    rows = sorted({(int(b), int(t)) for b, t in zip(r.integers(0, 4, 256), r.integers(0, 4096, 256))})
    rows += [(b, t) for b in range(4) for t in (0, 63, 64, 4095)]
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, 64, True, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(got), want, torch.bfloat16, mask)


def test_prefill_routed_long_context_and_block32():
    case("prefill_routed B=1 T=16384 bs=64 k=8")
    _routed_case(1, 16384, 12, 4, 64, 64, 8, seed=1005)
    case("prefill_routed B=4 T=4096 bs=32 k=4")
    _routed_case(4, 4096, 12, 4, 64, 32, 4, seed=1001)


def test_prefill_routed_four_heads_per_group_at_the_largest_block_count():
    # R = 4 takes 64-token windows; 1024 blocks of 64 keys (T = 65536)
    case("prefill_routed R=4 B=1 T=65536 bs=64 k=8")
    _routed_case(1, 65536, 16, 4, 64, 64, 8, seed=1013)


def test_prefill_routed_block32_at_the_largest_block_count():
    # 1024 blocks of 32 keys (T = 32768): 128-token windows with the most
    # blocks the set-up holds; routed == route + prefill, sampled rows against
    # the oracle
    case("prefill_routed B=1 T=32768 bs=32 k=4")
    T, bs, k = 32768, 32, 4
    x, sel, n, got = _routed_case(1, T, 12, 4, 64, bs, k, seed=1011)
    r = np.random.default_rng(11)
    ts = sorted({int(t) for t in r.integers(0, T, 48)} | {0, 31, 32, 16384, T - 32, T - 1})
    sel, n = sel.cpu().numpy(), n.cpu().numpy()
    protos = O.compress(np32(x["k"]), bs)
    f = np32(x["forecast"])
    for t in ts:
        _, _, s_o, n_o = O.route(f[:, t:t + 1], protos, bs, k, True, score_pos0=t, query_pos0=t)
        assert np.array_equal(n[:, :, t], n_o[:, :, 0]) and np.array_equal(sel[:, :, t], s_o[:, :, 0]), f"row {t}"
    rows = [(0, t) for t in ts]
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel, n, bs, True, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(got), want, torch.bfloat16, mask)


@pytest.mark.parametrize("bs", [64, 32])
def test_prefill_routed_small_top_k_and_short_lengths(bs):
    # top-k below the kernel's eight slots, top-k above the block count, single
    # tokens, one and two blocks, ragged tails
    for T, k in ((1, 8), (2, 1), (bs - 1, 3), (bs, 8), (bs + 1, 2), (2 * bs + 1, 8), (5 * bs - 1, 1), (300, 5)):
        case(f"prefill_routed T={T} bs={bs} k={k}")
        _routed_case(2, T, 12, 4, 64, bs, k, seed=500 + T + k)


def test_prefill_routed_fp32_forecast():
    case("prefill_routed fp32 forecast")
    _routed_case(2, 1000, 12, 4, 64, 64, 8, seed=420, fdtype=torch.float32)
    _routed_case(1, 600, 12, 4, 64, 32, 4, seed=421, fdtype=torch.float32, causal=False)


def test_prefill_routed_strided_views():
    # q / k / v as views of one packed projection output, the forecast a view
    # of a wider buffer: the one-launch kernel reads them through their strides
    case("prefill_routed strided views")
    B, T, Hq, Hkv, D, bs, k = 2, 700, 12, 4, 64, 64, 8
    x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=torch.bfloat16, seed=440)
    packed = torch.cat([x["q"], x["k"], x["v"]], dim=2).to(DEV)      # [B, T, Hq + 2 Hkv, D]
    q, kk, v = packed[:, :, :Hq], packed[:, :, Hq:Hq + Hkv], packed[:, :, Hq + Hkv:]
    wide = torch.zeros(B, T, Hkv, 2 * D, dtype=torch.bfloat16, device=DEV)
    wide[..., :D] = x["forecast"].to(DEV)
    f = wide[..., :D]
    protos = sparda.compress(kk, bs)
    got, sel, n = sparda.prefill_routed(q, kk, v, f, protos, bs, k, want_sel=True)
    _, _, sel_w, n_w = sparda.route(f.contiguous(), protos, bs, k, want_topk=False, want_sel=True)
    want = sparda.prefill(q.contiguous(), kk.contiguous(), v.contiguous(), sel_w, n_w, bs)
    torch.cuda.synchronize()
    assert torch.equal(sel, sel_w) and torch.equal(n, n_w)
    assert torch.equal(got, want)
    # lists wider than the kernel's ten entries: -1 padding as the router writes it
    got2, sel2, n2 = sparda.prefill_routed(q, kk, v, f, protos, bs, k, want_sel=True, sel_cap=13)
    _, _, sel_w2, n_w2 = sparda.route(f.contiguous(), protos, bs, k, want_topk=False, want_sel=True, sel_cap=13)
    torch.cuda.synchronize()
    assert torch.equal(sel2, sel_w2) and torch.equal(n2, n_w2) and torch.equal(got2, want)


def test_prefill_routed_two_launch_shapes():
    # shapes outside the one-launch kernel: top-k above 8, 16-key blocks,
    # D = 128, fp32 q/k/v, D = 32 (router then prefill through the hand-off
    # lists)
    case("prefill_routed two-launch shapes")
    _routed_case(1, 1000, 12, 4, 64, 64, 16, seed=430)
    _routed_case(1, 500, 12, 4, 64, 16, 4, seed=431)
    _routed_case(1, 300, 4, 1, 128, 32, 3, seed=432)
    _routed_case(1, 400, 12, 4, 64, 64, 8, seed=433, dtype=torch.float32)
    _routed_case(2, 333, 8, 2, 32, 16, 2, seed=434)


# ---------------------------------------------------------------------------
# decode step
# ---------------------------------------------------------------------------

def _decode_case(B, S, Hq, Hkv, D, bs, k, dtype, routing, seed, use_forecast=True, capacity=None):
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=dtype, seed=seed, capacity=capacity)
    d = {n: t.to(DEV) for n, t in x.items()}
    f = d["forecast"] if use_forecast else None
    out, ex = sparda.decode(d["q"], d["k_cache"], d["v_cache"], S, f, bs, k, routing=routing,
                            want_protos=True, want_sel=True)
    torch.cuda.synchronize()
    kc = np32(x["k_cache"])
    sel_o, n_o, _ = O.decode_selection(kc, S, np32(x["forecast"]) if use_forecast else None, bs, k, routing)
    assert np.array_equal(ex["n_sel"].cpu().numpy(), n_o)
    assert np.array_equal(ex["sel"].cpu().numpy(), sel_o)
    want = O.attention_decode(np32(x["q"]), kc, np32(x["v_cache"]), S, sel_o, n_o, bs)
    assert_close_out(np32(out), want, dtype)
    return d, out, ex


@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_decode_16k_cache(routing):
    # decode at 16K: B=8, cache [8,16384,4,64] bf16, 256 blocks, k=8 + sink + current
    case(f"decode 16K {routing}")
    d, out, ex = _decode_case(8, 16384, 12, 4, 64, 64, 8, torch.bfloat16, routing, seed=1002)
    assert np.array_equal(ex["protos"].cpu().numpy(), O.compress(np32(d["k_cache"]), 64))
    # a second call (nothing survives a call in the workspace) is identical
    out2 = sparda.decode(d["q"], d["k_cache"], d["v_cache"], 16384, d["forecast"], 64, 8, routing=routing)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_decode_between_256_and_512_blocks(routing):
    # 313 blocks: the selection runs on eight key registers per lane
    case(f"decode S=20000 {routing}")
    _decode_case(2, 20000, 12, 4, 64, 64, 8, torch.bfloat16, routing, seed=20000)


def test_decode_beyond_1024_blocks():
    # 1563 blocks: 64 key registers per lane
    case("decode S=100000 absolute")
    _decode_case(1, 100000, 12, 4, 64, 64, 8, torch.bfloat16, "absolute", seed=100000)


@pytest.mark.parametrize("S", [1, 63, 64, 65, 600, 1000, 5000])
def test_decode_lengths_fp32(S):
    case(f"decode fp32 S={S}")
    _decode_case(2, S, 12, 4, 64, 64, 8, torch.float32, "absolute", seed=S, capacity=S + 7)


def test_decode_static_window_and_dense_fallback():
    case("decode static + dense")
    _decode_case(3, 5000, 12, 4, 64, 64, 8, torch.bfloat16, "reference", seed=11, use_forecast=False)
    _decode_case(3, 600, 12, 4, 64, 64, 8, torch.bfloat16, "absolute", seed=12)  # NB=10 <= k+2


def test_decode_cached_prototypes_match():
    case("decode cached prototypes")
    x = synth.decode_inputs(2, 3000, 12, 4, 64, dtype=torch.bfloat16, seed=13)
    d = {n: t.to(DEV) for n, t in x.items()}
    out1, ex = sparda.decode(d["q"], d["k_cache"], d["v_cache"], 3000, d["forecast"], 64, 8,
                             routing="absolute", want_protos=True, want_sel=True)
    out2, ex2 = sparda.decode(d["q"], d["k_cache"], d["v_cache"], 3000, d["forecast"], 64, 8,
                              routing="absolute", protos_in=ex["protos"], want_sel=True)
    assert torch.equal(ex["sel"], ex2["sel"]) and torch.equal(out1, out2)


@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_decode_block32_reference_default_config(routing):
    # the reference's default configuration (configs/base.yaml:19-20): 32-key
    # blocks, top-4, on the matrix-core decode; ragged lengths and a cache short
    # enough that every block is attended
    case(f"decode bs=32 k=4 {routing}")
    _decode_case(8, 16384, 12, 4, 64, 32, 4, torch.bfloat16, routing, seed=1102)
    _decode_case(3, 5001, 12, 4, 64, 32, 4, torch.bfloat16, routing, seed=1103)
    _decode_case(2, 150, 12, 4, 64, 32, 4, torch.bfloat16, routing, seed=1104)  # NB=5 <= k+2


def test_decode_reference_geometry():
    # 8 q heads / 2 kv heads, D=32, bs=16, k=2 (tests/test_sparse_attention.py:14-30)
    case("decode D=32 bs=16 R=4")
    _decode_case(1, 53, 8, 2, 32, 16, 2, torch.float32, "reference", seed=14, capacity=128)
    _decode_case(1, 53, 8, 2, 32, 16, 2, torch.float32, "absolute", seed=15, capacity=128)
