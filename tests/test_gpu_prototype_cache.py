"""GPU parity of the cached-prototype decode: block sums of a device KV cache
kept current across steps, decode selection from the sums, attention over the
selected blocks in place.

Block sums / prototypes and selections are compared exactly (against
sparda.compress, the fused decode step and the oracle); attention outputs
within max-abs 2e-2 / mean-abs 2e-3 (bf16) or 1e-4 (fp32).
"""

import pytest
import torch

import sparda
from sparda import synth
from model.attention import HipSparseAttention, KVCache, PrototypeKVCache
from model.config import ModelConfig
from model.rope import RotaryEmbedding
from oracle import sparda_oracle as O
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("S,bs,dtype", [(4096, 64, torch.bfloat16), (5000, 64, torch.bfloat16),
                                        (333, 16, torch.float32)])
def test_block_sums_equal_compress_bit_exact(S, bs, dtype):
    case(f"block sums S={S} bs={bs} {dtype}")
    g = torch.Generator().manual_seed(S)
    k = torch.randn(2, S, 4, 64, generator=g).to(dtype).to(DEV)
    nb = (S + bs - 1) // bs
    sums = torch.full((2, nb + 3, 4, 64), float("nan"), device=DEV)
    sparda.block_sums(k, 0, S, bs, sums)
    protos = sparda.compress(k, bs)
    assert torch.equal(sums[:, :nb] / bs, protos)
    assert (sums[:, :nb] / bs).cpu().numpy().tobytes() == O.compress(np32(k), bs).tobytes()
    assert torch.isnan(sums[:, nb:]).all()  # blocks past the range untouched


def test_prototype_cache_incremental_updates_equal_one_shot():
    case("PrototypeKVCache incremental updates")
    bs = 64
    cache = PrototypeKVCache(2, 1200, 4, 64, DEV, torch.bfloat16, block_size=bs)
    g = torch.Generator().manual_seed(7)
    k = torch.randn(2, 1100, 4, 64, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(2, 1100, 4, 64, generator=g).to(torch.bfloat16).to(DEV)
    cache.update(k[:, :1000], v[:, :1000])
    for t in range(1000, 1100):  # one token at a time, crossing blocks 15 -> 17
        cache.update(k[:, t:t + 1], v[:, t:t + 1])
    # single-token appends leave the current block to the next decode launch
    assert cache.current_block_stale
    cache.refresh_sums()
    fresh = torch.zeros_like(cache.block_sums)
    sparda.block_sums(cache.k, 0, 1100, bs, fresh)
    nb = (1100 + bs - 1) // bs
    assert torch.equal(cache.block_sums[:, :nb], fresh[:, :nb])
    assert torch.equal(cache.block_sums[:, :nb] / bs, sparda.compress(k, bs))


@pytest.mark.parametrize("routing", ["reference", "absolute"])
@pytest.mark.parametrize("S", [5000, 16384])
def test_cached_selection_and_attention_equal_fused_decode(routing, S):
    case(f"cached-prototype decode S={S} {routing}")
    B, Hq, Hkv, D, bs, k = 4, 12, 4, 64, 64, 8
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=torch.bfloat16, seed=31)
    d = {n: t.to(DEV) for n, t in x.items()}
    out_f, ex = sparda.decode(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], bs, k, routing=routing,
                              want_sel=True)
    nb = (d["k_cache"].shape[1] + bs - 1) // bs
    sums = torch.zeros((B, nb, Hkv, D), device=DEV)
    sparda.block_sums(d["k_cache"], 0, S, bs, sums)
    sel, n = sparda.select_decode(d["forecast"], sums, S, S - 1, bs, k, routing=routing)
    out_c = sparda.decode_selected(d["q"], d["k_cache"], d["v_cache"], S, bs, sel, n)
    torch.cuda.synchronize()
    assert torch.equal(n, ex["n_sel"])
    for b in range(B):
        for g in range(Hkv):
            m = int(n[b, g])
            assert torch.equal(sel[b, g, :m], ex["sel"][b, g, :m])
    assert_close_out(np32(out_c), np32(out_f), torch.bfloat16, what="cached vs fused decode")
    want, sel_o, n_o = O.decode_step(np32(d["q"]), np32(d["k_cache"]), np32(d["v_cache"]), S,
                                     np32(d["forecast"]), bs, k, routing)
    assert (n.cpu().numpy() == n_o).all()
    assert_close_out(np32(out_c), want, torch.bfloat16, what="cached decode vs oracle")


@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_backend_decode_through_prototype_cache_equals_plain_cache(routing):
    case(f"HipSparseAttention with PrototypeKVCache {routing}")
    cfg = ModelConfig(block_size=64, top_k_blocks=8, context_length=4096, decode_routing=routing)
    torch.manual_seed(3)
    attn = HipSparseAttention(cfg, layer_idx=1).to(DEV).eval()
    rot = RotaryEmbedding(cfg.head_dim, 4096).to(DEV)
    plain = KVCache(1, 4096, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32)
    proto = PrototypeKVCache(1, 4096, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32, block_size=64)
    T = 1500
    x = torch.randn(1, T + 70, cfg.n_embd, device=DEV)
    f = torch.randn(1, T + 70, cfg.forecast_heads, cfg.forecast_dim, device=DEV)
    with torch.no_grad():
        a = attn(x[:, :T], rot, kv_cache=plain, forecast_vector=f[:, :T])
        b = attn(x[:, :T], rot, kv_cache=proto, forecast_vector=f[:, :T])
        assert torch.equal(a, b)
        for t in range(T, T + 70):  # crosses a block boundary (1536)
            a = attn(x[:, t:t + 1], rot, kv_cache=plain, forecast_vector=f[:, t:t + 1])
            b = attn(x[:, t:t + 1], rot, kv_cache=proto, forecast_vector=f[:, t:t + 1])
            assert_close_out(np32(b), np32(a), torch.float32, what=f"step {t}")
    nb = (T + 70 + 63) // 64
    assert torch.equal(proto.block_sums[:, :nb] / 64, sparda.compress(proto.k[:, :T + 70], 64))


@pytest.mark.parametrize("routing", ["reference", "absolute"])
@pytest.mark.parametrize("S,dtype", [(16384, torch.bfloat16), (16448, torch.bfloat16), (5000, torch.float32),
                                     (300, torch.bfloat16), (20000, torch.bfloat16), (40000, torch.bfloat16),
                                     (100000, torch.bfloat16)])
@pytest.mark.parametrize("bs,k", [(64, 8), (32, 4)])
def test_decode_sums_equals_separate_selection_and_attention(routing, S, dtype, bs, k):
    case(f"decode_sums (selection inside the attention launch) S={S} {dtype} {routing} bs={bs}")
    B, Hq, Hkv, D = 4, 12, 4, 64
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=dtype, seed=41)
    d = {n: t.to(DEV) for n, t in x.items()}
    nb = (S + bs - 1) // bs
    sums = torch.zeros((B, nb + 5, Hkv, D), device=DEV)
    sparda.block_sums(d["k_cache"], 0, S, bs, sums)
    sel, n = sparda.select_decode(d["forecast"], sums, S, S - 1, bs, k, routing=routing)
    want = sparda.decode_selected(d["q"], d["k_cache"], d["v_cache"], S, bs, sel, n)
    out, sel4, n4 = sparda.decode_sums(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], sums, bs, k,
                                       routing=routing, want_sel=True)
    torch.cuda.synchronize()
    assert torch.equal(n4, n) and torch.equal(sel4, sel)
    if nb > k + 2:  # the same list through the same attention: bit-equal
        assert torch.equal(out, want)
    else:           # every block: decode_selected takes its own wavefront split
        assert_close_out(np32(out), np32(want), dtype, what="dense fallback")
    # at a device-held position, bounded by the cache capacity
    pos = torch.full((1,), S - 1, dtype=torch.int64, device=DEV)
    out_d = sparda.decode_sums(d["q"], d["k_cache"], d["v_cache"], d["k_cache"].shape[1], d["forecast"], sums, bs,
                               k, routing=routing, pos_dev=pos)
    assert torch.equal(out_d, out)


def test_head_major_cache_layout_gives_the_same_decode():
    # the kernels take element strides: a head-major cache ([B,Hkv,S,D] storage,
    # each (head, block) one contiguous 8 KiB run) decodes exactly as the
    # reference's token-major [B,S,Hkv,D] one
    case("decode over a head-major (block-contiguous) cache")
    B, S, Hq, Hkv, D, bs, k = 2, 5000, 12, 4, 64, 64, 8
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=torch.bfloat16, seed=43)
    d = {n: t.to(DEV) for n, t in x.items()}
    hk = d["k_cache"].transpose(1, 2).contiguous().transpose(1, 2)
    hv = d["v_cache"].transpose(1, 2).contiguous().transpose(1, 2)
    assert hk.stride() == (Hkv * S * D, D, S * D, 1)
    for routing in ("reference", "absolute"):
        a = sparda.decode(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], bs, k, routing=routing)
        b = sparda.decode(d["q"], hk, hv, S, d["forecast"], bs, k, routing=routing)
        assert torch.equal(a, b)
    sa = torch.zeros((B, (S + bs - 1) // bs, Hkv, D), device=DEV)
    sb = torch.zeros_like(sa)
    sparda.block_sums(d["k_cache"], 0, S, bs, sa)
    sparda.block_sums(hk, 0, S, bs, sb)
    assert torch.equal(sa, sb)
    a = sparda.decode_sums(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], sa, bs, k, routing="absolute")
    b = sparda.decode_sums(d["q"], hk, hv, S, d["forecast"], sb, bs, k, routing="absolute")
    assert torch.equal(a, b)


@pytest.mark.parametrize("S,dtype", [(5000, torch.bfloat16), (4096, torch.bfloat16), (4097, torch.bfloat16),
                                     (300, torch.bfloat16), (2000, torch.float32)])
def test_decode_sums_updating_the_current_block(S, dtype):
    # the launch that recomputes the current block's sums first equals a
    # separate block_sums update followed by the plain launch, bit for bit,
    # and leaves the sums equal to a fresh computation
    case(f"decode_sums update_current S={S} {dtype}")
    B, Hq, Hkv, D, bs, k = 3, 12, 4, 64, 64, 8
    x = synth.decode_inputs(B, S, Hq, Hkv, D, dtype=dtype, seed=47)
    d = {n: t.to(DEV) for n, t in x.items()}
    nb = (S + bs - 1) // bs
    cb = (S - 1) // bs
    fresh = torch.zeros((B, nb + 2, Hkv, D), device=DEV)
    sparda.block_sums(d["k_cache"], 0, S, bs, fresh)
    stale = torch.zeros_like(fresh)
    sparda.block_sums(d["k_cache"], 0, S - 1, bs, stale)  # the sums before token S-1 was appended
    if cb * bs < S - 1:
        assert not torch.equal(stale[:, cb], fresh[:, cb])
    for routing in ("reference", "absolute"):
        want, sel_w, n_w = sparda.decode_sums(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], fresh, bs, k,
                                              routing=routing, want_sel=True)
        sums = stale.clone()
        got, sel_g, n_g = sparda.decode_sums(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], sums, bs, k,
                                             routing=routing, want_sel=True, update_current=True)
        torch.cuda.synchronize()
        assert torch.equal(sums, fresh)
        assert torch.equal(n_g, n_w) and torch.equal(sel_g, sel_w)
        assert torch.equal(got, want)
        # at a device-held position
        sums = stale.clone()
        pos = torch.full((1,), S - 1, dtype=torch.int64, device=DEV)
        got_d = sparda.decode_sums(d["q"], d["k_cache"], d["v_cache"], d["k_cache"].shape[1], d["forecast"], sums,
                                   bs, k, routing=routing, pos_dev=pos, update_current=True)
        torch.cuda.synchronize()
        assert torch.equal(sums, fresh) and torch.equal(got_d, want)
