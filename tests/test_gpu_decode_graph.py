"""GPU parity of the decode steps at a device-held position and of the
generation loop replayed from one captured HIP graph.

Entries that read the position from device memory are compared bit for bit
with their host-length counterparts (same kernels, same launch shapes); the
window mode's every-block fallback on a short cache with the dense decode
within max-abs 2e-2 / mean-abs 2e-3 (bf16) or 1e-4 (fp32). The replayed
generation loop is compared with the eager cached-prototype decode of the same
model: logits of every step bit for bit, sampled tokens identical. A replayed
step's forecast-routed layers are checked against the oracle from the caches,
block sums and the q / forecast the replay left behind: the selection
bit-exact, the attention within the bf16 bar. A parameter changed in place or
replaced between steps makes the next step record again from the new weights.
"""

import numpy as np
import pytest
import torch

import sparda
from model.attention import PrototypeKVCache
from model.config import ModelConfig
from model.decode_graph import GraphDecoder
from model.model import SparDAResearchModel
from helpers import assert_close_out, np32
from oracle import sparda_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def _pos(p):
    return torch.full((1,), p, dtype=torch.int64, device=DEV)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_device_position_ops_equal_host_length_ops(dtype, routing):
    case(f"device-position ops {dtype} {routing}")
    B, Smax, Hq, Hkv, D, bs, k = 2, 2048, 12, 4, 64, 64, 8
    g = torch.Generator().manual_seed(11)
    kc = torch.randn(B, Smax, Hkv, D, generator=g).to(dtype).to(DEV)
    vc = torch.randn(B, Smax, Hkv, D, generator=g).to(dtype).to(DEV)
    q = torch.randn(B, Hq, D, generator=g).to(dtype).to(DEV)
    f = torch.randn(B, Hkv, 64, generator=g).to(DEV)
    nb = Smax // bs
    sums = torch.zeros((B, nb, Hkv, D), device=DEV)
    sparda.block_sums(kc, 0, Smax, bs, sums)
    for p in (0, 63, 64, 639, 640, 641, 700, 1535, 2047):
        case(f"  position {p}")
        pos = _pos(p)
        j = p // bs
        # current-block sums: [j*bs, p], the other blocks untouched
        got = torch.full_like(sums, float("nan"))
        sparda.append_at(kc, None, pos, bs, got)
        want = torch.full_like(sums, float("nan"))
        sparda.block_sums(kc, j * bs, p - j * bs + 1, bs, want)
        assert torch.equal(got[:, j], want[:, j])
        assert torch.isnan(got[:, :j]).all() and torch.isnan(got[:, j + 1:]).all()
        # append of a new row at p: the caches gain it, the sums equal a fresh sum
        kn = torch.randn(B, 1, Hkv, D, generator=g).to(dtype).to(DEV)
        vn = torch.randn(B, 1, Hkv, D, generator=g).to(dtype).to(DEV)
        k2, v2, s2 = kc.clone(), vc.clone(), torch.full_like(sums, float("nan"))
        sparda.append_at(k2, v2, pos, bs, s2, kn, vn)
        k3, v3 = kc.clone(), vc.clone()
        k3[:, p:p + 1], v3[:, p:p + 1] = kn, vn
        assert torch.equal(k2, k3) and torch.equal(v2, v3)
        sparda.block_sums(k3, j * bs, p - j * bs + 1, bs, want)
        assert torch.equal(s2[:, j], want[:, j])
        # selection from the sums
        s_d, n_d = sparda.select_decode_at(f, sums, pos, Smax, bs, k, routing=routing)
        s_h, n_h = sparda.select_decode(f, sums, p + 1, p, bs, k, routing=routing)
        assert torch.equal(n_d, n_h) and torch.equal(s_d, s_h)
        # attention over the selection
        o_d = sparda.decode_at(q, kc, vc, pos, bs, s_d, n_d)
        o_h = sparda.decode_selected(q, kc, vc, p + 1, bs, s_h, n_h)
        assert torch.equal(o_d, o_h)
        # static window (no forecast): the fused decode's window mode
        o_w = sparda.decode_at(q, kc, vc, pos, bs, window=k)
        o_r = sparda.decode(q, kc, vc, p + 1, None, bs, k)
        if j + 1 > k + 2:
            assert torch.equal(o_w, o_r)
        else:  # every block: the fused decode's dense mode (its own wavefront split)
            assert_close_out(np32(o_w), np32(o_r), dtype, what=f"window fallback p={p}")
        # every block
        o_a = sparda.decode_at(q, kc, vc, pos, bs, window=0)
        o_b = sparda.decode_selected(q, kc, vc, p + 1, bs)
        assert_close_out(np32(o_a), np32(o_b), dtype, what=f"dense p={p}")
    torch.cuda.synchronize()


@pytest.mark.parametrize("routing", ["reference", "absolute"])
@pytest.mark.parametrize("bs", [64, 32])
def test_decode_at_carrying_a_prefetch_equals_separate_launches(routing, bs):
    # the attention launch that carries the next layer's prefetch (selection
    # with lookahead + copy from the arena) must leave the attention output,
    # the selection and the compact buffers exactly as decode_at,
    # select_decode_at(lookahead) and fetch_at do as separate launches
    case(f"decode_at carrying the next layer's prefetch, bs={bs} {routing}")
    B, Smax, Hq, Hkv, D, k = 2, 2048, 12, 4, 64, 8
    cap, bf = k + 2, torch.bfloat16
    g = torch.Generator().manual_seed(13)
    kc = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    vc = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    q = torch.randn(B, Hq, D, generator=g).to(bf).to(DEV)
    f = torch.randn(B, Hkv, 64, generator=g).to(bf if bs == 64 else torch.float32).to(DEV)
    kn = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    vn = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    arena = sparda.OffloadArena(B, Smax, Hkv, D, bf)
    arena.append(kn, vn, 0)
    nb = Smax // bs
    own_sums = torch.zeros((B, nb, Hkv, D), device=DEV)
    sparda.block_sums(kc, 0, Smax, bs, own_sums)

    def outputs():
        return (torch.full((B, Hkv, cap), 7, dtype=torch.int32, device=DEV),
                torch.full((B, Hkv), 7, dtype=torch.int32, device=DEV),
                torch.full((B, Hkv, cap, bs, D), 3.0, dtype=bf, device=DEV),
                torch.full((B, Hkv, cap, bs, D), 3.0, dtype=bf, device=DEV))

    for p in (0, 1, bs - 1, bs, bs + 1, 639, 640, 641, 1535, 2047):
        case(f"  position {p}")
        pos = _pos(p)
        sums = torch.zeros((B, nb, Hkv, D), device=DEV)
        if p > 0:
            sparda.block_sums(kn, 0, p, bs, sums)
        s1, n1, k1, v1 = outputs()
        sparda.select_decode_at(f, sums, pos, Smax, bs, k, routing=routing, sel=s1, n_sel=n1, lookahead=True)
        arena.fetch_at(s1, n1, bs, pos, k1, v1)
        sa, na = sparda.select_decode_at(f, own_sums, pos, Smax, bs, k, routing=routing)
        for mode in ("list", "every block"):
            s2, n2, k2, v2 = outputs()
            spec = dict(arena=arena, forecast=f, block_sums=sums, top_k=k, routing=routing, sel=s2, n_sel=n2,
                        k_dst=k2, v_dst=v2)
            if mode == "list":
                o_plain = sparda.decode_at(q, kc, vc, pos, bs, sa, na)
                o_carry = sparda.decode_at(q, kc, vc, pos, bs, sa, na, prefetch=spec)
            else:
                o_plain = sparda.decode_at(q, kc, vc, pos, bs, window=0)
                o_carry = sparda.decode_at(q, kc, vc, pos, bs, window=0, prefetch=spec)
            assert torch.equal(o_carry, o_plain), f"attention output, {mode}, p={p}"
            assert torch.equal(n2, n1) and torch.equal(s2, s1), f"selection, {mode}, p={p}"
            assert torch.equal(k2, k1) and torch.equal(v2, v1), f"fetched blocks, {mode}, p={p}"
    # only the matrix-core attention carries a prefetch: fp32 is refused before any launch
    s2, n2, k2, v2 = outputs()
    spec = dict(arena=arena, forecast=f, block_sums=own_sums, top_k=k, routing=routing, sel=s2, n_sel=n2,
                k_dst=k2, v_dst=v2)
    with pytest.raises(ValueError):
        sparda.decode_at(q.float(), kc.float(), vc.float(), _pos(100), bs, window=0, prefetch=spec)
    torch.cuda.synchronize()
    arena.close()


@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_prefetch_split_over_the_append_and_attention_launches(routing):
    # the next layer's selection carried by this layer's arena append (stage 1)
    # and its copy by this layer's attention launch (stage 2): the selection,
    # the fetched blocks, the append (arena rows and block sums) and the
    # attention output equal the separate launches'
    case(f"prefetch stages over the append and attention launches, {routing}")
    B, Smax, Hq, Hkv, D, bs, k = 2, 2048, 12, 4, 64, 64, 8
    cap, bf = k + 2, torch.bfloat16
    g = torch.Generator().manual_seed(14)
    f = torch.randn(B, Hkv, 64, generator=g).to(bf).to(DEV)
    q = torch.randn(B, Hq, D, generator=g).to(bf).to(DEV)
    kn = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    vn = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    kc = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    vc = torch.randn(B, Smax, Hkv, D, generator=g).to(bf).to(DEV)
    nxt = sparda.OffloadArena(B, Smax, Hkv, D, bf)
    nxt.append(kn, vn, 0)
    C, Fh = 256, 512  # a small feed-forward to carry shares of the copy
    xf = torch.randn(B, 1, C, generator=g).to(bf).to(DEV)
    wgu = (torch.randn(2 * Fh, C, generator=g) * 0.05).to(bf).to(DEV)
    wdn = (torch.randn(C, Fh, generator=g) * 0.05).to(bf).to(DEV)
    cur_a = sparda.OffloadArena(B, Smax, Hkv, D, bf)   # appended to plainly
    cur_b = sparda.OffloadArena(B, Smax, Hkv, D, bf)   # appended to by the launch carrying the selection
    cur_a.append(kc[:, :1500], vc[:, :1500], 0)
    cur_b.append(kc[:, :1500], vc[:, :1500], 0)
    nb = Smax // bs

    def outputs():
        return (torch.full((B, Hkv, cap), 7, dtype=torch.int32, device=DEV),
                torch.full((B, Hkv), 7, dtype=torch.int32, device=DEV),
                torch.full((B, Hkv, cap, bs, D), 3.0, dtype=bf, device=DEV),
                torch.full((B, Hkv, cap, bs, D), 3.0, dtype=bf, device=DEV))

    sums_a = torch.zeros((B, nb, Hkv, D), device=DEV)
    sums_b = torch.zeros((B, nb, Hkv, D), device=DEV)
    cur_a.rebuild_sums(1500, bs, sums_a)
    cur_b.rebuild_sums(1500, bs, sums_b)
    for p in (1500, 1535, 1536, 1537, 2047):
        case(f"  position {p}")
        pos = _pos(p)
        sums = torch.zeros((B, nb, Hkv, D), device=DEV)
        sparda.block_sums(kn, 0, p, bs, sums)
        s1, n1, k1, v1 = outputs()
        sparda.select_decode_at(f, sums, pos, Smax, bs, k, routing=routing, sel=s1, n_sel=n1, lookahead=True)
        nxt.fetch_at(s1, n1, bs, pos, k1, v1)
        s2, n2, k2, v2 = outputs()
        spec = dict(arena=nxt, forecast=f, block_sums=sums, top_k=k, routing=routing, sel=s2, n_sel=n2,
                    k_dst=k2, v_dst=v2)
        row_k, row_v = kc[:, p:p + 1], vc[:, p:p + 1]
        cur_a.append_at(row_k, row_v, pos, bs, sums_a)
        cur_b.append_at(row_k, row_v, pos, bs, sums_b, prefetch={**spec, "stage": 1}, max_len=Smax)
        torch.cuda.synchronize()
        assert torch.equal(n2, n1) and torch.equal(s2, s1), f"selection at {p}"
        assert (k2 == 3.0).all() and (v2 == 3.0).all(), "stage 1 copies nothing"
        assert torch.equal(sums_b, sums_a), f"block sums at {p}"
        # the carrying layer attends densely over its own (resident) cache here
        o_plain = sparda.decode_at(q, kc, vc, pos, bs, window=0)
        o_carry = sparda.decode_at(q, kc, vc, pos, bs, window=0, prefetch={**spec, "stage": 2})
        assert torch.equal(o_carry, o_plain), f"attention output at {p}"
        assert torch.equal(k2, k1) and torch.equal(v2, v1), f"fetched blocks at {p}"
        assert torch.equal(s2, s1) and torch.equal(n2, n1), "stage 2 leaves the selection"
        # the copy in three shares: share 0 by the attention launch, shares 1
        # and 2 by the two feed-forward launches; each copies its slots only
        _, _, k3, v3 = outputs()
        spec3 = {**spec, "k_dst": k3, "v_dst": v3, "stage": 2, "parts": 3}
        o3 = sparda.decode_at(q, kc, vc, pos, bs, window=0, prefetch={**spec3, "part": 0})
        torch.cuda.synchronize()
        assert torch.equal(o3, o_plain)
        mine = torch.zeros(cap, dtype=torch.bool)
        mine[0::3] = True
        assert torch.equal(k3[:, :, mine], k1[:, :, mine]) and (k3[:, :, ~mine] == 3.0).all(), "share 0"
        y_plain = sparda.ffn_decode(xf, wgu, wdn, 1e-5)
        y = sparda.ffn_decode(xf, wgu, wdn, 1e-5, prefetch=({**spec3, "part": 1}, {**spec3, "part": 2}),
                              pos_dev=pos, block_size=bs)
        torch.cuda.synchronize()
        assert torch.equal(y, y_plain), f"feed-forward output at {p}"
        assert torch.equal(k3, k1) and torch.equal(v3, v1), f"blocks fetched in three shares at {p}"
    L = 2048
    assert torch.equal(cur_a.k_host[:, :L], cur_b.k_host[:, :L]) and torch.equal(cur_a.v_host[:, :L],
                                                                                  cur_b.v_host[:, :L])
    for a in (nxt, cur_a, cur_b):
        a.close()


def test_device_positions_are_clamped_into_range():
    case("device-position clamping")
    B, Smax, Hq, Hkv, D, bs, k = 1, 1000, 12, 4, 64, 64, 8
    g = torch.Generator().manual_seed(12)
    kc = torch.randn(B, Smax, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(B, Smax, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    f = torch.randn(B, Hkv, 64, generator=g).to(DEV)
    sums = torch.zeros((B, (Smax + bs - 1) // bs, Hkv, D), device=DEV)
    sparda.block_sums(kc, 0, Smax, bs, sums)
    hi, lo = _pos(Smax + 500), _pos(-7)
    last, first = _pos(Smax - 1), _pos(0)
    for a, b in ((hi, last), (lo, first)):
        sa, na = sparda.select_decode_at(f, sums, a, Smax, bs, k)
        sb_, nb_ = sparda.select_decode_at(f, sums, b, Smax, bs, k)
        assert torch.equal(sa, sb_) and torch.equal(na, nb_)
        assert torch.equal(sparda.decode_at(q, kc, vc, a, bs, sa, na), sparda.decode_at(q, kc, vc, b, bs, sb_, nb_))
        assert torch.equal(sparda.decode_at(q, kc, vc, a, bs, window=k), sparda.decode_at(q, kc, vc, b, bs, window=k))
        x = torch.full_like(sums, 3.0)
        y = torch.full_like(sums, 3.0)
        sparda.append_at(kc, None, a, bs, x)
        sparda.append_at(kc, None, b, bs, y)
        assert torch.equal(x, y)


def test_produce_at_device_position_equals_host_position():
    case("produce at a device position")
    torch.manual_seed(13)
    B, C, nq, nkv, nf = 3, 768, 768, 256, 256
    x = (torch.randn(B, 1, C) * 0.5).to(torch.bfloat16).to(DEV)
    w = (torch.randn(nq + 2 * nkv + nf, C) * 0.02).to(torch.bfloat16).to(DEV)
    from model.rope import rope_tables
    cos, sin = rope_tables(64, 2048, 10000.0)
    cos, sin = cos.to(DEV), sin.to(DEV)
    for p in (0, 1, 777, 2047):
        want = sparda.produce(x, w, nq, nkv, nf, 1e-5, cos, sin, pos0=p)
        got = sparda.produce(x, w, nq, nkv, nf, 1e-5, cos, sin, pos_dev=_pos(p))
        for a, b in zip(got, want):
            assert torch.equal(a, b)
    # positions past the tables are clamped to the last row
    want = sparda.produce(x, w, nq, nkv, nf, 1e-5, cos, sin, pos0=2047)
    got = sparda.produce(x, w, nq, nkv, nf, 1e-5, cos, sin, pos_dev=_pos(5000))
    for a, b in zip(got, want):
        assert torch.equal(a, b)


def _model(mode, routing, n_layer=3, ctx=2048, fused_ffn=False):
    backend = {"forecast": "hip_sparse", "static": "static_sparse", "dense": "dense"}[mode]
    cfg = ModelConfig(n_layer=n_layer, context_length=ctx, block_size=64, top_k_blocks=8, decode_routing=routing,
                      attention_backend=backend, fused_producer=True, fused_ffn=fused_ffn, norm_eps=1e-5)
    torch.manual_seed(21)
    return SparDAResearchModel(cfg).to(DEV, torch.bfloat16).eval(), cfg


@pytest.mark.parametrize("mode,routing,fused_ffn", [("forecast", "reference", False), ("forecast", "absolute", False),
                                                    ("static", "reference", False), ("forecast", "absolute", True)])
def test_graph_replayed_steps_equal_eager_cached_decode(mode, routing, fused_ffn):
    case(f"graph-replayed decode steps, {mode} {routing} fused_ffn={fused_ffn}")
    model, cfg = _model(mode, routing, fused_ffn=fused_ffn)
    B, T0, n, cap = 2, 900, 100, 1100  # 15 blocks at the start, crossing 960 and 1024
    g = torch.Generator().manual_seed(22)
    ids = torch.randint(0, cfg.vocab_size, (B, T0 + n), generator=g).to(DEV)
    caches = [PrototypeKVCache(B, cap, cfg.n_kv_head, cfg.head_dim, DEV, torch.bfloat16, block_size=64)
              for _ in range(cfg.n_layer)]
    gd = GraphDecoder(model, B, cap)
    with torch.no_grad():
        want = [model(ids[:, :T0], kv_caches=caches)["logits"][:, -1]]
        for t in range(T0, T0 + n):
            want.append(model(ids[:, t:t + 1], kv_caches=caches)["logits"][:, -1])
        got = [gd.prefill(ids[:, :T0])]
        for t in range(T0, T0 + n):
            got.append(gd.step(ids[:, t:t + 1]).clone())
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"step {i}: max diff {(a.float() - b.float()).abs().max().item()}"
    for c, e in zip(gd.caches, caches):
        assert c.current_len == e.current_len == T0 + n
        assert torch.equal(c.k[:, :T0 + n], e.k[:, :T0 + n]) and torch.equal(c.v[:, :T0 + n], e.v[:, :T0 + n])
        e.refresh_sums()  # eager layers without a forecast left their last single-token block deferred
        assert torch.equal(c.block_sums, e.block_sums)


def test_graph_generation_equals_eager_generation_and_replays_after_reset():
    case("graph generation vs eager generation")
    model, cfg = _model("forecast", "absolute")
    B, T0, n, cap = 2, 700, 80, 1024
    g = torch.Generator().manual_seed(23)
    prompt = torch.randint(0, cfg.vocab_size, (B, T0), generator=g).to(DEV)
    gd = GraphDecoder(model, B, cap)
    for temperature in (0.0, 0.8):
        caches = [PrototypeKVCache(B, cap, cfg.n_kv_head, cfg.head_dim, DEV, torch.bfloat16, block_size=64)
                  for _ in range(cfg.n_layer)]
        torch.manual_seed(5)
        want = model.generate(prompt, max_new_tokens=n, temperature=temperature, top_k=50, kv_caches=caches)
        torch.manual_seed(5)
        got = gd.generate(prompt, max_new_tokens=n, temperature=temperature, top_k=50)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"temperature {temperature}"
    assert gd.graph is not None  # the second generation replayed the step recorded by the first


@pytest.mark.parametrize("routing", ["absolute", "reference"])
def test_graph_replayed_offload_steps_equal_eager_async_offload(routing):
    case(f"graph-replayed offload decode (prefetch on a side stream), {routing}")
    from model.attention import AsyncOffloadedKVCache, KVCache
    cfg = ModelConfig(n_layer=3, context_length=2048, block_size=64, top_k_blocks=8, decode_routing=routing,
                      attention_backend="async_offload", fused_producer=True, fused_ffn=routing == "absolute",
                      norm_eps=1e-5)
    torch.manual_seed(24)
    model = SparDAResearchModel(cfg).to(DEV, torch.bfloat16).eval()
    B, T0, n, cap = 2, 900, 100, 1100
    g = torch.Generator().manual_seed(25)
    ids = torch.randint(0, cfg.vocab_size, (B, T0 + n), generator=g).to(DEV)
    caches = [KVCache(B, cap, cfg.n_kv_head, cfg.head_dim, DEV, torch.bfloat16)] + [
        AsyncOffloadedKVCache(B, cap, cfg.n_kv_head, cfg.head_dim, DEV, torch.bfloat16, block_size=64)
        for _ in range(cfg.n_layer - 1)]
    gd = GraphDecoder(model, B, cap, overlap=True)
    serial = GraphDecoder(model, B, cap, overlap=False)
    fused = GraphDecoder(model, B, cap)  # the prefetch carried by the previous layer's attention launch
    assert fused.overlap == "fused"
    with torch.no_grad():
        want = [model(ids[:, :T0], kv_caches=caches)["logits"][:, -1]]
        for t in range(T0, T0 + n):
            want.append(model(ids[:, t:t + 1], kv_caches=caches)["logits"][:, -1])
        got = [gd.prefill(ids[:, :T0])]
        got_s = [serial.prefill(ids[:, :T0])]
        got_f = [fused.prefill(ids[:, :T0])]
        for t in range(T0, T0 + n):
            got.append(gd.step(ids[:, t:t + 1]).clone())
            got_s.append(serial.step(ids[:, t:t + 1]).clone())
            got_f.append(fused.step(ids[:, t:t + 1]).clone())
    torch.cuda.synchronize()
    for i, (a, b, d, c) in enumerate(zip(got, got_s, got_f, want)):
        assert torch.equal(a, c), f"step {i}: max diff {(a.float() - c.float()).abs().max().item()}"
        assert torch.equal(b, c), f"serial step {i}"
        assert torch.equal(d, c), f"fused-prefetch step {i}"
    L = T0 + n
    for dec in (gd, fused):
        assert torch.equal(dec.caches[0].k[:, :L], caches[0].k[:, :L])
        for c, e in zip(dec.caches[1:], caches[1:]):
            assert c.current_len == e.current_len == L
            assert torch.equal(c.cpu_k[:, :L], e.cpu_k[:, :L]) and torch.equal(c.cpu_v[:, :L], e.cpu_v[:, :L])
            assert torch.equal(c.block_sums(64), e.block_sums(64))


def test_graph_decoder_sixteen_sequences_and_capacity_limit():
    case("graph-replayed decode, 16 sequences (the largest decode-shape batch), up to the capacity")
    model, cfg = _model("forecast", "absolute", n_layer=2, fused_ffn=True)
    B, T0, cap = 16, 700, 712
    g = torch.Generator().manual_seed(26)
    ids = torch.randint(0, cfg.vocab_size, (B, cap), generator=g).to(DEV)
    caches = [PrototypeKVCache(B, cap, cfg.n_kv_head, cfg.head_dim, DEV, torch.bfloat16, block_size=64)
              for _ in range(cfg.n_layer)]
    gd = GraphDecoder(model, B, cap)
    with torch.no_grad():
        model(ids[:, :T0], kv_caches=caches)
        gd.prefill(ids[:, :T0])
        for t in range(T0, cap):
            want = model(ids[:, t:t + 1], kv_caches=caches)["logits"][:, -1]
            got = gd.step(ids[:, t:t + 1])
            assert torch.equal(got, want), f"position {t}"
        with pytest.raises(ValueError):
            gd.step(ids[:, :1])  # the caches are full


@pytest.mark.parametrize("backend,routing", [("hip_sparse", "reference"), ("hip_sparse", "absolute"),
                                             ("async_offload", "reference"), ("async_offload", "absolute")])
def test_graph_replayed_step_against_the_oracle(backend, routing):
    # layers 1 and 2 are routed by the forecast of the layer before them; at
    # each checked step their q, routing forecast and attention output are
    # read from the replay's own buffers
    case(f"graph-replayed step vs the oracle, {backend} {routing}")
    cfg = ModelConfig(n_layer=3, context_length=2048, block_size=64, top_k_blocks=8, decode_routing=routing,
                      attention_backend=backend, fused_producer=True, fused_ffn=True, norm_eps=1e-5)
    torch.manual_seed(27)
    model = SparDAResearchModel(cfg).to(DEV, torch.bfloat16).eval()
    B, T0, n, cap, bs, k = 2, 900, 70, 1100, 64, 8
    Hkv = cfg.n_kv_head
    g = torch.Generator().manual_seed(28)
    ids = torch.randint(0, cfg.vocab_size, (B, T0 + n), generator=g).to(DEV)
    gd = GraphDecoder(model, B, cap, taps=(1, 2))
    checked = 0
    with torch.no_grad():
        gd.prefill(ids[:, :T0])
        for t in range(T0, T0 + n):
            gd.step(ids[:, t:t + 1])
            if t not in (T0, 959, 960, T0 + n - 1):  # first step, the last row of a block, a new block, last
                continue
            torch.cuda.synchronize()
            S = gd.length
            for i in (1, 2):
                case(f"  position {S - 1}, layer {i}")
                c, tap = gd.caches[i], gd.tapped[i]
                f = tap["f"].reshape(B, Hkv, -1)
                if backend == "hip_sparse":
                    kc, vc = np32(c.k[:, :S]), np32(c.v[:, :S])
                    sel_o, n_o, _ = O.decode_selection(kc, S, np32(f), bs, k, routing)
                    # the replay's block sums select what the oracle selects from the keys
                    sel, n_sel = sparda.select_decode(f, c.block_sums, S, S - 1, bs, k, routing=routing)
                else:
                    kc, vc = c.cpu_k[:, :S].float().numpy(), c.cpu_v[:, :S].float().numpy()
                    # the prefetch selected before the token at S - 1 was appended
                    sel_o, n_o = O.prefetch_selection(kc, S - 1, S - 1, np32(f), bs, k, routing)
                    sel, n_sel = tap["sel"], tap["n_sel"]
                assert np.array_equal(n_sel.cpu().numpy(), n_o)
                assert np.array_equal(sel.cpu().numpy(), sel_o)
                want = O.attention_decode(np32(tap["q"]), kc, vc, S, sel_o, n_o, bs)
                assert_close_out(np32(tap["out"]), want, torch.bfloat16, what=f"layer {i} at {S - 1}")
                checked += 1
    assert checked == 8


def test_graph_records_again_after_a_weight_change():
    case("graph-replayed decode after in-place and replacing weight changes")
    model, cfg = _model("forecast", "absolute", fused_ffn=True)
    B, T0, n, cap = 2, 700, 30, 1024
    g = torch.Generator().manual_seed(29)
    ids = torch.randint(0, cfg.vocab_size, (B, T0 + n), generator=g).to(DEV)
    caches = [PrototypeKVCache(B, cap, cfg.n_kv_head, cfg.head_dim, DEV, torch.bfloat16, block_size=64)
              for _ in range(cfg.n_layer)]
    gd = GraphDecoder(model, B, cap)
    graphs = []
    with torch.no_grad():
        model(ids[:, :T0], kv_caches=caches)
        gd.prefill(ids[:, :T0])
        for t in range(T0, T0 + n):
            if t == T0 + 10:
                # in place: the folded producer, FFN and head weights are stale
                model.layers[1].attn_norm.weight.mul_(1.5)
                model.layers[2].ffn_norm.weight.mul_(0.75)
                model.final_norm.weight.mul_(1.25)
                model.embeddings.weight[int(ids[0, t + 1])].mul_(1.5)
            if t == T0 + 20:
                # replaced: the recorded step would read the old tensor's memory
                w = model.layers[0].ffn.w_down.weight
                model.layers[0].ffn.w_down.weight = torch.nn.Parameter(w * 1.25)
                model.layers[1].attention.wo.weight = torch.nn.Parameter(model.layers[1].attention.wo.weight * 0.8)
            want = model(ids[:, t:t + 1], kv_caches=caches)["logits"][:, -1]
            got = gd.step(ids[:, t:t + 1])
            if not graphs or graphs[-1] is not gd.graph:
                graphs.append(gd.graph)
            assert torch.equal(got, want), f"position {t}: max diff {(got.float() - want.float()).abs().max().item()}"
    assert len(graphs) == 3  # recorded at the first step and after each change
