"""GPU parity of the fused producer (RMSNorm + q / k / v / forecast
projections + RoPE in one kernel) against a plain PyTorch fp32 restatement of
model/norm.py:15-21, the projections, model/forecast.py:30-40 and
model/rope.py:34-65; and of the model with the fused producer against the
model without it. Tolerances: max-abs 2e-2 / mean-abs 2e-3 (bf16 outputs)."""

import pytest
import torch

import sparda
from model.attention import KVCache
from model.config import ModelConfig
from model.model import SparDAResearchModel
from model.rope import rope_tables
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def _reference(x, w_stack, norm_w, eps, cos, sin, pos0, nq, nkv):
    """fp32: RMSNorm, stacked projection, rotate-half RoPE of the q and k heads."""
    xf = x.float()
    normed = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * norm_w.float()
    y = normed @ w_stack.float().t()
    B, T, _ = x.shape
    q, k, v, f = torch.split(y, [nq, nkv, nkv, y.shape[-1] - nq - 2 * nkv], dim=-1)
    c = cos[pos0:pos0 + T][None, :, None, :]
    s = sin[pos0:pos0 + T][None, :, None, :]

    def rot(t):
        t = t.view(B, T, -1, 64)
        a, b = t[..., :32], t[..., 32:]
        return torch.cat((a * c - b * s, b * c + a * s), dim=-1)

    return rot(q), rot(k), v.view(B, T, -1, 64), f.view(B, T, -1, 64)


@pytest.mark.parametrize("B,T,pos0,f_dtype", [(2, 300, 5, torch.bfloat16), (1, 1024, 0, torch.float32),
                                               (4, 1, 4000, torch.bfloat16), (1, 1, 0, torch.bfloat16),
                                               (16, 1, 77, torch.float32), (8, 2, 9, torch.bfloat16),
                                               (17, 1, 3, torch.bfloat16)])
def test_produce_matches_fp32_reference(B, T, pos0, f_dtype):
    case(f"produce B={B} T={T} pos0={pos0} {f_dtype}")
    g = torch.Generator().manual_seed(11 + T)
    C, nq, nkv, nf, eps = 768, 768, 256, 256, 1e-5
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(nq + 2 * nkv + nf, C, generator=g)).to(torch.bfloat16)
    norm_w = (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16)
    cos, sin = rope_tables(64, 4096)
    w_fold = (w.float() * norm_w.float()[None, :]).to(torch.bfloat16)
    q, k, v, f = sparda.produce(x.to(DEV), w_fold.to(DEV), nq, nkv, nf, eps, cos.to(DEV), sin.to(DEV),
                                pos0=pos0, f_dtype=f_dtype)
    want = _reference(x, w, norm_w, eps, cos, sin, pos0, nq, nkv)
    for got, ref, name in zip((q, k, v, f), want, "qkvf"):
        assert got.shape == ref.shape, name
        assert_close_out(np32(got), ref.numpy(), torch.bfloat16, what=f"produce {name}")


def _pair(fused, **kw):
    # dense attention: forecast routing is a discrete top-k of F, so the bf16
    # rounding differences between the fused and the unfused F may flip
    # near-tied blocks; without routing the logits differ only by rounding
    cfg = ModelConfig(n_layer=2, context_length=2048, block_size=64, top_k_blocks=8, attention_backend="dense",
                      norm_eps=1e-5, decode_routing="absolute", fused_producer=fused, **kw)
    torch.manual_seed(5)
    return SparDAResearchModel(cfg).to(DEV, torch.bfloat16).eval()


def _no_less_accurate(fused, plain, ref, what):
    """The fused producer rounds at other places than the unfused sequence (the
    folded weight instead of the normalised activations, RoPE in fp32), so both
    bf16 models are compared with the same weights run in fp32: the fused one
    must be as accurate as the unfused one (mean and max error within 25%)."""
    f = np32(fused).astype("float64")
    p = np32(plain).astype("float64")
    r = np32(ref).astype("float64")
    ef, ep = abs(f - r), abs(p - r)
    assert ef.mean() <= 1.25 * ep.mean() + 1e-5, f"{what}: mean error {ef.mean():.3e} vs unfused {ep.mean():.3e}"
    assert ef.max() <= 1.25 * ep.max() + 1e-3, f"{what}: max error {ef.max():.3e} vs unfused {ep.max():.3e}"


def test_model_with_fused_producer_matches_unfused():
    case("model forward and decode with / without the fused producer (dense attention), vs fp32")
    plain, fused = _pair(False), _pair(True)
    fused.load_state_dict(plain.state_dict())
    ref = _pair(False).float()
    ref.load_state_dict({k: v.float() for k, v in plain.state_dict().items()})
    probe = torch.zeros(1, 1, 768, device=DEV, dtype=torch.bfloat16)
    assert not fused.layers[1]._use_fused_producer(probe, None)  # autograd on: unfused
    with torch.no_grad():
        assert fused.layers[1]._use_fused_producer(probe, None)
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, plain.config.vocab_size, (2, 700), generator=g).to(DEV)
    with torch.no_grad():
        _no_less_accurate(fused(ids)["logits"], plain(ids)["logits"], ref(ids)["logits"], "prefill logits")
        caches = [[KVCache(2, 800, 4, 64, DEV, dt) for _ in range(2)]
                  for dt in (torch.bfloat16, torch.bfloat16, torch.float32)]
        for m, c in zip((plain, fused, ref), caches):
            m(ids[:, :650], kv_caches=c)
        for t in range(650, 660):
            a, b, r = (m(ids[:, t:t + 1], kv_caches=c)["logits"] for m, c in zip((plain, fused, ref), caches))
            _no_less_accurate(b, a, r, f"decode logits {t}")
        # the fused weight follows parameter updates
        for m in (plain, fused, ref):
            m.layers[1].attn_norm.weight.mul_(1.5)
        _no_less_accurate(fused(ids[:, :300])["logits"], plain(ids[:, :300])["logits"],
                          ref(ids[:, :300])["logits"], "logits after a weight update")


def _ffn_reference(x, wg, wu, wd, norm_w, eps):
    """fp32: x + w_down(silu(w_gate(n)) * w_up(n)), n = RMSNorm(x) * norm_w."""
    xf = x.float()
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * norm_w.float()
    g = n @ wg.float().t()
    u = n @ wu.float().t()
    return xf + (torch.nn.functional.silu(g) * u) @ wd.float().t()


@pytest.mark.parametrize("M,C,F", [(1, 768, 2048), (16, 768, 2048), (5, 256, 512), (3, 1024, 128)])
def test_ffn_decode_matches_fp32_reference(M, C, F):
    case(f"ffn_decode M={M} C={C} F={F}")
    torch.manual_seed(M * 1000 + C)
    x = (torch.randn(M, 1, C) * 0.7).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(F, C) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(F, C) * 0.02).to(torch.bfloat16).to(DEV)
    wd = (torch.randn(C, F) * 0.02).to(torch.bfloat16).to(DEV)
    nw = (1.0 + 0.1 * torch.randn(C)).to(torch.bfloat16).to(DEV)
    wgu = (torch.cat([wg.float(), wu.float()]) * nw.float()[None, :]).to(torch.bfloat16)
    got = sparda.ffn_decode(x, wgu, wd, 1e-5)
    ref = _ffn_reference(x, wg, wu, wd, nw, 1e-5)
    assert_close_out(np32(got), ref.cpu().numpy(), torch.bfloat16, what="ffn_decode")
    # (B, T) = (M, 1) and (1, M) rows are the same rows
    got2 = sparda.ffn_decode(x.view(1, M, C), wgu, wd, 1e-5)
    assert torch.equal(got2.view(M, 1, C), got)


def test_model_with_fused_ffn_matches_unfused():
    case("cached decode with / without the fused FFN (dense attention), vs fp32")
    plain, fused = _pair(True), _pair(True, fused_ffn=True)
    fused.load_state_dict(plain.state_dict())
    ref = _pair(False).float()
    ref.load_state_dict({k: v.float() for k, v in plain.state_dict().items()})
    probe = torch.zeros(2, 1, 768, device=DEV, dtype=torch.bfloat16)
    assert not fused.layers[1]._use_fused_ffn(probe)  # autograd on: unfused
    with torch.no_grad():
        assert fused.layers[1]._use_fused_ffn(probe)
        assert not fused.layers[1]._use_fused_ffn(torch.zeros(2, 9, 768, device=DEV, dtype=torch.bfloat16))
    g = torch.Generator().manual_seed(10)
    ids = torch.randint(0, plain.config.vocab_size, (2, 700), generator=g).to(DEV)
    with torch.no_grad():
        caches = [[KVCache(2, 800, 4, 64, DEV, dt) for _ in range(2)]
                  for dt in (torch.bfloat16, torch.bfloat16, torch.float32)]
        for m, c in zip((plain, fused, ref), caches):
            m(ids[:, :650], kv_caches=c)
        for t in range(650, 660):
            a, b, r = (m(ids[:, t:t + 1], kv_caches=c)["logits"] for m, c in zip((plain, fused, ref), caches))
            _no_less_accurate(b, a, r, f"decode logits {t}")
        for m in (plain, fused, ref):
            m.layers[0].ffn_norm.weight.mul_(1.5)  # the folded weight follows parameter updates
        a, b, r = (m(ids[:, 660:661], kv_caches=c)["logits"] for m, c in zip((plain, fused, ref), caches))
        _no_less_accurate(b, a, r, "decode logits after a weight update")
        # the folded output head follows the final norm and the tied table (one
        # row scaled: the next token's embedding and that vocabulary column)
        tok = int(ids[0, 661])
        head = fused._folded_head()
        for m in (plain, fused, ref):
            m.final_norm.weight.mul_(1.25)
            m.embeddings.weight[tok].mul_(1.5)
        a, b, r = (m(ids[:, 661:662], kv_caches=c)["logits"] for m, c in zip((plain, fused, ref), caches))
        assert fused._folded_head() is not head
        _no_less_accurate(b, a, r, "decode logits after a head update")


@pytest.mark.parametrize("M,K,N", [(1, 768, 768), (8, 768, 768), (16, 2048, 256), (3, 128, 16)])
def test_rows_residual_op(M, K, N):
    # res + a . w^T with the projection rounded to bf16 first, against the
    # same two roundings around an fp32 product
    g = torch.Generator().manual_seed(M * 131 + K)
    a = torch.randn(M, 1, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(DEV)
    res = torch.randn(M, 1, N, generator=g).to(torch.bfloat16).to(DEV)
    got = sparda.rows_residual(a, w, res)
    proj = (a.float().reshape(M, K) @ w.float().T).to(torch.bfloat16)
    want = (res.float().reshape(M, N) + proj.float()).to(torch.bfloat16)
    diff = (got.reshape(M, N).float() - want.float()).abs()
    # accumulation order only: within one bf16 rounding step of the projection and the sum
    tol = want.float().abs() * 2 ** -7 + proj.float().abs() * 2 ** -7 + 1e-3
    assert bool((diff <= tol).all()), f"max diff {diff.max().item()}"


def test_produce_writes_the_cache_rows():
    # the cache-writing producer equals produce_at followed by a row copy into
    # the caches; rows outside position p stay untouched
    case_B, C, nq, nkv, nf = 4, 768, 768, 256, 256
    g = torch.Generator().manual_seed(61)
    x = torch.randn(case_B, 1, C, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(nq + 2 * nkv + nf, C, generator=g) / C ** 0.5).to(torch.bfloat16).to(DEV)
    cos, sin = rope_tables(64, 300)
    cos, sin = cos.to(DEV), sin.to(DEV)
    for p in (0, 77, 299):
        pos = torch.full((1,), p, dtype=torch.int64, device=DEV)
        kc = torch.randn(case_B, 300, nkv // 64, 64, device=DEV).to(torch.bfloat16)
        vc = torch.randn_like(kc)
        k0, v0 = kc.clone(), vc.clone()
        q1, k1, v1, f1 = sparda.produce(x, w, nq, nkv, nf, 1e-5, cos, sin, pos_dev=pos)
        q2, k2, v2, f2 = sparda.produce(x, w, nq, nkv, nf, 1e-5, cos, sin, pos_dev=pos, k_cache=kc, v_cache=vc)
        torch.cuda.synchronize()
        assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2) and torch.equal(f1, f2)
        assert torch.equal(kc[:, p], k1[:, 0]) and torch.equal(vc[:, p], v1[:, 0])
        rest = [t for t in range(300) if t != p]
        assert torch.equal(kc[:, rest], k0[:, rest]) and torch.equal(vc[:, rest], v0[:, rest])


@pytest.mark.parametrize("M,C,N", [(1, 768, 32000), (8, 768, 4096), (16, 1024, 160)])
def test_norm_gemv_op(M, C, N):
    # final RMSNorm + output projection, against the fp32 product of the
    # folded weight divided by rms(x), one bf16 rounding
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, 1, C, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, C, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    nw = (1.0 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).to(DEV)
    wf = (w.float() * nw.float()[None, :]).to(torch.bfloat16)
    got = sparda.norm_gemv(x, wf, 1e-6)
    xf = x.float().reshape(M, C)
    want = (xf @ wf.float().T) / torch.sqrt((xf * xf).mean(-1, keepdim=True) + 1e-6)
    diff = (got.reshape(M, N).float() - want).abs()
    tol = want.abs() * 2 ** -7 + 1e-3
    assert bool((diff <= tol).all()), f"max diff {diff.max().item()}"
    # against the unfolded composition RMSNorm(x) * g @ W^T in fp32: the folded
    # weight's one bf16 rounding (unit roundoff 2^-8) bounds the extra error by
    # 2^-8 * |x / rms| . |W * g|
    xn = xf / torch.sqrt((xf * xf).mean(-1, keepdim=True) + 1e-6)
    wg = w.float() * nw.float()[None, :]
    want2 = xn @ wg.T
    diff2 = (got.reshape(M, N).float() - want2).abs()
    tol2 = want2.abs() * 2 ** -7 + 2 ** -8 * (xn.abs() @ wg.abs().T) + 1e-3
    assert bool((diff2 <= tol2).all()), f"unfolded: max diff {diff2.max().item()}"
