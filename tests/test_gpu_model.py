"""GPU checks of the backends and the model harness: backend outputs against
the oracle on the same projected inputs, decode bookkeeping with a KV cache,
the offload backends against the GPU-resident one, and the prefetch state
protocol of the reference's async tests (tests/test_async_offload.py)."""

import numpy as np
import pytest
import torch

import sparda
from model.attention import (AsyncOffloadedKVCache, HipAsyncOffloadAttention, HipOffloadAttention,
                             HipSparseAttention, KVCache, OffloadedKVCache)
from model.config import ModelConfig
from model.model import SparDAResearchModel
from model.rope import RotaryEmbedding
from oracle import sparda_oracle as O
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def small_config(**kw):
    # the reference's test geometry (tests/test_sparse_attention.py:14-30; test_async_offload.py:20-40)
    base = dict(vocab_size=1000, n_layer=4, n_embd=256, n_head=8, n_kv_head=2, head_dim=32, ffn_dim=512,
                forecast_heads=2, forecast_dim=32, context_length=512, block_size=16, top_k_blocks=2)
    base.update(kw)
    return ModelConfig(**base)


def _project(attn, rotary, x, offset=0):
    B, T, _ = x.shape
    xq = attn.wq(x).view(B, T, attn.n_head, attn.head_dim)
    xk = attn.wk(x).view(B, T, attn.n_kv_head, attn.head_dim)
    xv = attn.wv(x).view(B, T, attn.n_kv_head, attn.head_dim)
    xq, xk = rotary(xq, xk, offset=offset)
    return xq, xk, xv


def _wo64(attn, o):
    return o @ attn.wo.weight.detach().double().cpu().numpy().T


@pytest.mark.parametrize("dtype,bs,k", [(torch.float32, 64, 8), (torch.bfloat16, 64, 8), (torch.bfloat16, 32, 4)])
def test_sparse_backend_prefill_matches_oracle(dtype, bs, k):
    # (32, 4): the reference's default block configuration (configs/base.yaml)
    case(f"HipSparseAttention prefill {dtype} bs={bs} k={k}")
    cfg = ModelConfig(block_size=bs, top_k_blocks=k, context_length=1024)
    torch.manual_seed(0)
    attn = HipSparseAttention(cfg, layer_idx=1).to(DEV, dtype).eval()
    rot = RotaryEmbedding(cfg.head_dim, 1024).to(DEV)
    x = torch.randn(1, 1024, cfg.n_embd, device=DEV).to(dtype)
    f = torch.randn(1, 1024, cfg.forecast_heads, cfg.forecast_dim, device=DEV).to(dtype)
    with torch.no_grad():
        out = attn(x, rot, forecast_vector=f)
        xq, xk, xv = _project(attn, rot, x)
    sel, n = O.prefill_selection(np32(xk), np32(f), bs, k)
    rows = [(0, t) for t in range(0, 1024, 7)]
    o = O.attention_prefill(np32(xq), np32(xk), np32(xv), sel, n, bs, rows=rows)
    idx = [t for _, t in rows]
    want = _wo64(attn, o[0, idx])
    tol_dtype = torch.bfloat16 if dtype == torch.bfloat16 else torch.float32
    # wo in the layer's dtype adds its own rounding on top of the attention's
    got = np32(out)[0, idx]
    if dtype == torch.float32:
        assert np.abs(got - want).max() < 1e-4
    else:
        assert_close_out(got, want, tol_dtype, what="prefill+wo")


def test_sparse_backend_decode_with_kv_cache_matches_oracle():
    case("HipSparseAttention decode with KVCache")
    cfg = ModelConfig(block_size=64, top_k_blocks=8, context_length=4096, decode_routing="absolute")
    torch.manual_seed(1)
    attn = HipSparseAttention(cfg, layer_idx=1).to(DEV).eval()
    rot = RotaryEmbedding(cfg.head_dim, 4096).to(DEV)
    cache = KVCache(1, 4096, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32)
    T = 1500
    x = torch.randn(1, T + 3, cfg.n_embd, device=DEV)
    f = torch.randn(1, T + 3, cfg.forecast_heads, cfg.forecast_dim, device=DEV)
    with torch.no_grad():
        attn(x[:, :T], rot, kv_cache=cache, forecast_vector=f[:, :T])
        for t in range(T, T + 3):
            out = attn(x[:, t:t + 1], rot, kv_cache=cache, forecast_vector=f[:, t:t + 1])
            assert cache.current_len == t + 1
            xq, _, _ = _project(attn, rot, x[:, t:t + 1], offset=t)
            S = t + 1
            kc, vc = np32(cache.k), np32(cache.v)
            sel, n, _ = O.decode_selection(kc, S, np32(f[:, t]), 64, 8, "absolute")
            o = O.attention_decode(np32(xq[:, 0]), kc, vc, S, sel, n, 64)
            assert np.abs(np32(out)[:, 0] - _wo64(attn, o)).max() < 1e-4


@pytest.mark.parametrize("routing", ["reference", "absolute"])
def test_offload_backend_equals_gpu_resident_backend(routing):
    case(f"offload vs resident {routing}")
    cfg = ModelConfig(block_size=64, top_k_blocks=8, context_length=4096, decode_routing=routing)
    torch.manual_seed(2)
    res = HipSparseAttention(cfg, layer_idx=1).to(DEV).eval()
    off = HipOffloadAttention(cfg, layer_idx=1).to(DEV).eval()
    off.load_state_dict(res.state_dict())
    rot = RotaryEmbedding(cfg.head_dim, 4096).to(DEV)
    c_res = KVCache(1, 4096, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32)
    c_off = OffloadedKVCache(1, 4096, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32)
    T = 2000
    x = torch.randn(1, T + 4, cfg.n_embd, device=DEV)
    f = torch.randn(1, T + 4, cfg.forecast_heads, cfg.forecast_dim, device=DEV)
    with torch.no_grad():
        # prefill: the offload backend attends densely over the prompt (as the reference's does)
        res(x[:, :T], rot, kv_cache=c_res, forecast_vector=None)
        off(x[:, :T], rot, kv_cache=c_off, forecast_vector=f[:, :T])
        for t in range(T, T + 4):
            a = res(x[:, t:t + 1], rot, kv_cache=c_res, forecast_vector=f[:, t:t + 1])
            b = off(x[:, t:t + 1], rot, kv_cache=c_off, forecast_vector=f[:, t:t + 1])
            assert torch.equal(a, b)
    torch.cuda.synchronize()
    assert torch.equal(c_off.cpu_k[:, :T + 4], c_res.k[:, :T + 4].cpu())
    assert c_off.total_transfer_calls == 4
    assert c_off.total_bytes_transferred == 4 * 2 * cfg.n_kv_head * 10 * 64 * cfg.head_dim * 4


def test_offloaded_cache_transfer_selected_blocks_known_answer():
    # restates tests/test_offload.py:32-76: blocks 0 and 1 of two heads, byte accounting
    case("OffloadedKVCache.transfer_selected_blocks")
    cache = OffloadedKVCache(1, 64, 2, 32, DEV, torch.float32)
    assert cache.current_len == 0 and cache.cpu_k.device.type == "cpu" and cache.cpu_k.is_pinned()
    k = torch.randn(1, 32, 2, 32, device=DEV)
    v = torch.randn(1, 32, 2, 32, device=DEV)
    assert cache.update(k, v) == 32
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu_k[:, :32], k.cpu())
    idx = torch.tensor([[[0], [1]]], device=DEV)
    gk, gv, nbytes = cache.transfer_selected_blocks(idx, 16)
    torch.cuda.synchronize()
    assert gk.shape == (1, 2, 16, 32)
    assert nbytes == (gk.numel() + gv.numel()) * gk.element_size() == cache.total_bytes_transferred
    assert torch.equal(gk[0, 0], k[0, 0:16, 0]) and torch.equal(gk[0, 1], k[0, 16:32, 1])
    assert torch.equal(gv[0, 1], v[0, 16:32, 1])


def test_async_cache_transfer_and_event():
    case("AsyncOffloadedKVCache.async_transfer_selected_blocks")
    cache = AsyncOffloadedKVCache(1, 64, 2, 32, DEV, torch.float32)
    k = torch.randn(1, 40, 2, 32, device=DEV)
    cache.update(k, k * 2)
    gk, gv, ev, nbytes = cache.async_transfer_selected_blocks(torch.tensor([[[2], [0]]], device=DEV), 16)
    torch.cuda.current_stream().wait_event(ev)
    assert gk.shape == (1, 2, 16, 32)
    # block 2 holds tokens 32..39; rows past current_len read as zeros
    assert torch.equal(gk[0, 0, :8], k[0, 32:40, 0]) and (gk[0, 0, 8:] == 0).all()
    assert torch.equal(gv[0, 1], 2 * k[0, 0:16, 1])
    assert nbytes == cache.total_bytes_transferred


def test_async_prefetch_protocol_and_parity_with_sync():
    # tests/test_async_offload.py:100-176: prefetch queued, consumed, and equal to the sync backend
    case("async prefetch protocol + parity")
    cfg = small_config()
    torch.manual_seed(42)
    sync_attn = HipOffloadAttention(cfg, layer_idx=1).to(DEV).eval()
    async_attn = HipAsyncOffloadAttention(cfg, layer_idx=1).to(DEV).eval()
    async_attn.load_state_dict(sync_attn.state_dict())
    rot = RotaryEmbedding(cfg.head_dim, 128).to(DEV)
    c_sync = OffloadedKVCache(1, 128, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32)
    c_async = AsyncOffloadedKVCache(1, 128, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32)
    prompt = torch.randn(1, 100, cfg.n_embd, device=DEV)
    with torch.no_grad():
        sync_attn(prompt, rot, kv_cache=c_sync)
        async_attn(prompt, rot, kv_cache=c_async)
        assert c_sync.current_len == c_async.current_len == 100
        for step in range(3):
            tok = torch.randn(1, 1, cfg.n_embd, device=DEV)
            fv = torch.randn(1, 1, cfg.forecast_heads, cfg.forecast_dim, device=DEV)
            assert async_attn.prefetch(fv, offload_cache=c_async) is True
            assert async_attn.prefetch_event is not None and async_attn.prefetched_gpu_k is not None
            a = sync_attn(tok, rot, kv_cache=c_sync, forecast_vector=fv)
            b = async_attn(tok, rot, kv_cache=c_async, forecast_vector=fv)
            assert async_attn.prefetch_event is None and async_attn.prefetched_gpu_k is None
            assert c_async.current_len == 101 + step
            # reference routing: both select {0..k-1} U {own}; same blocks, same kernel
            assert torch.allclose(a, b, atol=1e-4)
    # an empty cache cannot be prefetched
    empty = AsyncOffloadedKVCache(1, 16, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32)
    assert async_attn.prefetch(torch.randn(1, 1, 2, 32, device=DEV), empty) is False


def test_async_prefetch_absolute_matches_oracle_and_stale_prefetch_is_dropped():
    case("async prefetch absolute + stale")
    cfg = ModelConfig(block_size=64, top_k_blocks=8, context_length=4096, decode_routing="absolute")
    torch.manual_seed(3)
    attn = HipAsyncOffloadAttention(cfg, layer_idx=2).to(DEV, torch.bfloat16).eval()
    rot = RotaryEmbedding(cfg.head_dim, 4096).to(DEV)
    cache = AsyncOffloadedKVCache(2, 4096, cfg.n_kv_head, cfg.head_dim, DEV, torch.bfloat16, block_size=64)
    T = 3000
    x = torch.randn(2, T + 2, cfg.n_embd, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        attn(x[:, :T], rot, kv_cache=cache)
        fv = torch.randn(2, 1, cfg.forecast_heads, cfg.forecast_dim, device=DEV).to(torch.bfloat16)
        attn.track_overlap = True
        assert attn.prefetch(fv, cache)
        # the selection is written on the transfer stream: wait for its event before reading it here
        torch.cuda.current_stream().wait_event(attn.prefetch_event)
        sel = attn.prefetched_sel_indices.clone()
        out = attn(x[:, T:T + 1], rot, kv_cache=cache, forecast_vector=fv)
        xq, xk, xv = _project(attn, rot, x[:, T:T + 1], offset=T)
        torch.cuda.synchronize()
        kc, vc = np32(cache.cpu_k), np32(cache.cpu_v)
        sel_o, n_o = O.prefetch_selection(kc, T, T, np32(fv[:, 0]), 64, 8, "absolute")
        assert np.array_equal(sel.cpu().numpy(), sel_o)
        o = O.attention_decode(np32(xq[:, 0]), kc, vc, T + 1, sel_o, n_o, 64)
        assert_close_out(np32(out)[:, 0], _wo64(attn, o), torch.bfloat16, what="async decode + wo")
        st = attn.overlap_stats()
        assert st["steps"] == 1 and st["transfer_ms"] > 0 and 0.0 <= st["overlap"] <= 1.0
        # a prefetch issued for another cache length is not used
        assert attn.prefetch(fv, cache)
        cache.update(xk, xv)  # the cache moves on without the attention
        attn(x[:, T + 1:T + 2], rot, kv_cache=cache, forecast_vector=fv)
        assert attn.stale_prefetches == 1


@pytest.mark.parametrize("backend", ["hip_sparse", "dense", "static", "offload", "async_offload"])
def test_model_forward_and_cached_decode(backend):
    case(f"model {backend}")
    cfg = small_config(attention_backend=backend)
    torch.manual_seed(4)
    model = SparDAResearchModel(cfg).to(DEV).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, 80), device=DEV)
    with torch.no_grad():
        out = model(ids, return_forecasts=True)
        assert out["logits"].shape == (1, 80, cfg.vocab_size) and torch.isfinite(out["logits"]).all()
        assert len(out["forecasts"]) == cfg.n_layer
        if backend in ("offload", "async_offload"):
            cls = AsyncOffloadedKVCache if backend == "async_offload" else OffloadedKVCache
            caches = [cls(1, 128, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32) for _ in range(cfg.n_layer)]
        else:
            caches = [KVCache(1, 128, cfg.n_kv_head, cfg.head_dim, DEV, torch.float32) for _ in range(cfg.n_layer)]
        gen = model.generate(ids, max_new_tokens=5, temperature=0.0, kv_caches=caches)
        assert gen.shape == (1, 85) and all(c.current_len == 84 for c in caches)


def test_async_model_decode_matches_gpu_resident_model():
    # 12-layer-style stack at reduced size: async prefetch decode == GPU-resident sparse decode
    case("async model vs resident model")
    torch.manual_seed(5)
    cfg_a = small_config(attention_backend="async_offload", n_layer=3)
    cfg_r = small_config(attention_backend="offload", n_layer=3)
    ma = SparDAResearchModel(cfg_a).to(DEV).eval()
    mr = SparDAResearchModel(cfg_r).to(DEV).eval()
    mr.load_state_dict(ma.state_dict())
    ids = torch.randint(0, cfg_a.vocab_size, (1, 100), device=DEV)
    ca = [AsyncOffloadedKVCache(1, 160, 2, 32, DEV, torch.float32) for _ in range(3)]
    cr = [OffloadedKVCache(1, 160, 2, 32, DEV, torch.float32) for _ in range(3)]
    with torch.no_grad():
        la = ma(ids, kv_caches=ca)["logits"]
        lr = mr(ids, kv_caches=cr)["logits"]
        assert torch.allclose(la, lr, atol=1e-4)
        for _ in range(4):
            nxt = la[:, -1:].argmax(-1)
            la = ma(nxt, kv_caches=ca)["logits"]
            lr = mr(nxt, kv_caches=cr)["logits"]
            assert torch.allclose(la, lr, atol=1e-4)
    assert ma.layers[1].attention.stale_prefetches == 0
