"""C-ABI library checks that need no GPU: it loads, exports exactly what
include/sparda.h declares, and rejects bad arguments before any HIP call."""

import os
import re

import pytest

import sparda
from sparda import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sparda.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"SPARDA_API\s+[\w\s\*]+?\b(sparda_\w+)\s*\(", text)))


def test_library_loads_and_reports_version():
    lib = sparda.load()
    assert lib.sparda_version() == 100


def test_the_loaded_library_is_the_in_tree_build():
    # the mapping the process holds is the file next to the binding, unless
    # SPARDA_LIBRARY overrides it on purpose
    if os.environ.get("SPARDA_LIBRARY"):
        pytest.skip("SPARDA_LIBRARY overrides the library path")
    in_tree = os.path.join(ROOT, "local-research-small-language-model_amd", "sparda", "libsparda.so")
    sparda.load()
    maps = open("/proc/self/maps").read()
    mapped = {line.split()[-1] for line in maps.splitlines() if line.endswith("libsparda.so")}
    assert mapped and all(os.path.samefile(m, in_tree) for m in mapped), mapped


def test_every_declared_symbol_is_exported_and_bound():
    lib = sparda.load()
    syms = header_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in sparda.h but not exported"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"


def test_every_exported_symbol_is_declared():
    # the reverse: nothing the library exports (and the binding uses) is
    # missing from the header a C caller compiles against
    import subprocess
    syms = set(header_symbols())
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("nm not available")
    exported = set(re.findall(r"\b(sparda_\w+)$", out.stdout, flags=re.M))
    assert exported, "no sparda_* symbols found in the library"
    assert exported <= syms, f"exported but not declared in sparda.h: {sorted(exported - syms)}"
    assert set(_lib.SIGNATURES) <= syms, f"bound but not declared: {sorted(set(_lib.SIGNATURES) - syms)}"


def _expect(code, name, *args):
    with pytest.raises(sparda.SpardaArgumentError) as ei:
        _lib.call(name, *args)
    assert ei.value.code == code
    assert sparda.load().sparda_last_error()


def test_argument_errors_are_reported_before_any_hip_call():
    P = 4096  # any non-null value: validation fails before it is dereferenced
    _expect(-1, "sparda_compress", None, 0, 1, 1, 1, 1, 1, 1, 1, 1, P, None)
    _expect(-3, "sparda_compress", P, 7, 1, 1, 1, 1, 1, 1, 1, 1, P, None)
    _expect(-2, "sparda_compress", P, 1, 1, 0, 1, 1, 1, 1, 1, 1, P, None)
    _expect(-2, "sparda_route", P, 1, 1, 1, 1, P, 1, 1, 1, 48, 4, 8, 8, 1, 0, 0, 0.125, P, None, None, None, 0,
            None)  # Df=48 unsupported
    _expect(-2, "sparda_route", P, 1, 1, 1, 1, P, 1, 1, 1, 64, 4, 8, 33, 1, 0, 0, 0.125, P, None, None, None,
            0, None)  # top_k > 32
    _expect(-2, "sparda_route", P, 1, 1, 1, 1, P, 1, 1, 1, 64, 16, 8, 8, 1, 0, 0, 0.125, None, None, P, P, 9,
            None)  # sel_cap < k+2
    _expect(-6, "sparda_topk_scores", P, 1, 8, 2, 9, P, None)
    _expect(-6, "sparda_select_fixed", 7, 1, 1, 1, 1, 1, 1, 0, P, P, 4, None)
    _expect(-2, "sparda_prefill", P, 1, 1, 1, P, P, 1, 1, 1, 1, None, None, 0, 1, 16, 12, 5, 64, 64, 1, 0.125,
            P, 1, 1, None)  # Hq not a multiple of Hkv
    # prefill_routed: q, strides, k, v, kv strides, dtype, forecast, f_dtype, f strides, protos, Df, top_k,
    # route_scale, sel, n_sel, sel_cap, B, T, Hq, Hkv, D, bs, causal, scale, out, out strides, stream
    routed = lambda f, sel, n_sel, cap, top_k, protos=P: (
        P, 768, 768, 64, P, P, 256, 256, 64, 1, f, 1, 256, 256, 64, protos, 64, top_k, 0.125, sel, n_sel, cap,
        1, 1024, 12, 4, 64, 64, 1, 0.125, P, 768, 768, None)
    _expect(-1, "sparda_prefill_routed", *routed(None, None, None, 0, 8))        # no forecast
    _expect(-1, "sparda_prefill_routed", *routed(P, P, None, 10, 8))            # sel without n_sel
    _expect(-2, "sparda_prefill_routed", *routed(P, None, None, 0, 33))         # top_k > 32
    _expect(-2, "sparda_prefill_routed", *routed(P, P, P, 9, 8))                # sel_cap < top_k + 2
    _expect(-2, "sparda_prefill_routed", *routed(P, None, None, 0, 16))         # two launches need the lists
    _expect(-5, "sparda_prefill_routed", *routed(P, None, None, 0, 8, P + 4))   # unaligned prototypes
    _expect(-4, "sparda_decode", P, 1, 1, P, P, 8, 8, 8, 1, None, 0, 0, 0, 1, 128, 12, 4, 64, 64, 8, 0, 0.125,
            None, None, None, None, P, 1, None, 0, None)  # no workspace
    _expect(-4, "sparda_decode", P, 1, 1, P, P, 8, 8, 8, 1, None, 0, 0, 0, 1, 128, 12, 4, 64, 64, 8, 0, 0.125,
            None, None, None, None, P, 1, P * 2, 16, None)  # workspace too small
    _expect(-6, "sparda_decode", P, 1, 1, P, P, 8, 8, 8, 1, None, 0, 0, 0, 1, 128, 12, 4, 64, 64, 8, 5, 0.125,
            None, None, None, None, P, 1, P * 2, 1 << 20, None)  # unknown routing
    # x, x_st, w, M, C, Nq, Nk, Nf, eps, cos, sin, rope_len, T, pos_dev, q, k, v, f, f_dtype,
    # k_cache, v_cache, sb, st, sh, max_len, stream
    _expect(-1, "sparda_produce_cache_at", P, 768, P, 1, 768, 768, 256, 256, 1e-5, P, P, 64, 1, P, P, P, P, P, 1,
            None, P, 8, 8, 8, 64, None)  # no k_cache
    _expect(-2, "sparda_produce_cache_at", P, 768, P, 17, 768, 768, 256, 256, 1e-5, P, P, 64, 1, P, P, P, P, P, 1,
            P, P, 8, 8, 8, 64, None)  # M > 16
    # x, x_st, w, M, C, N, eps, out, out_st, stream
    _expect(-1, "sparda_norm_gemv", None, 768, P, 1, 768, 32000, 1e-6, P, 32000, None)
    _expect(-2, "sparda_norm_gemv", P, 768, P, 1, 768, 32001, 1e-6, P, 32001, None)   # N % 16
    _expect(-2, "sparda_norm_gemv", P, 2048, P, 1, 2048, 32000, 1e-6, P, 32000, None)  # C > 1024
    # a, a_st, w, M, K, N, res, res_st, out, out_st, stream
    _expect(-1, "sparda_rows_residual", None, 768, P, 1, 768, 768, P, 768, P, 768, None)
    _expect(-2, "sparda_rows_residual", P, 768, P, 17, 768, 768, P, 768, P, 768, None)   # M > 16
    _expect(-2, "sparda_rows_residual", P, 768, P, 1, 700, 768, P, 768, P, 768, None)   # K % 128
    _expect(-2, "sparda_rows_residual", P, 768, P, 1, 768, 760, P, 768, P, 768, None)   # N % 16
    _expect(-5, "sparda_rows_residual", P + 4, 768, P, 1, 768, 768, P, 768, P, 768, None)  # misaligned a


def test_chunked_entry_argument_errors():
    P = 4096
    # topk, width, B, H, T, bs, top_k, sel, n_sel, cap, stream
    _expect(-1, "sparda_select_chunked", P, 8, 1, 4, 1000, 64, 8, None, P, 10, None)      # no sel
    _expect(-2, "sparda_select_chunked", P, 9, 1, 4, 1000, 64, 8, P, P, 10, None)         # width > top_k
    _expect(-2, "sparda_select_chunked", P, 8, 1, 4, 1000, 64, 8, P, P, 9, None)          # cap < min(NB, k+2)
    _expect(-2, "sparda_select_chunked", P, 8, 1, 4, 4097 * 64, 64, 8, P, P, 10, None)    # more than 4096 blocks
    # q, strides, k, v, kv strides, dtype, topk, width, top_k, sel, n_sel, cap, B, T, Hq, Hkv, D, bs, scale,
    # out, out strides, stream
    ch = lambda topk, width, top_k, sel, n_sel, cap, T=1000, bs=64, Hq=12: (
        P, 768, 768, 64, P, P, 256, 256, 64, 1, topk, width, top_k, sel, n_sel, cap, 1, T, Hq, 4, 64, bs, 0.125,
        P, 768, 768, None)
    _expect(-1, "sparda_prefill_chunked", *ch(P, 8, 8, P, None, 10))                    # sel without n_sel
    _expect(-2, "sparda_prefill_chunked", *ch(P, 8, 33, None, None, 0))                 # top_k > 32
    _expect(-2, "sparda_prefill_chunked", *ch(P, 9, 8, None, None, 0))                  # width > top_k
    _expect(-2, "sparda_prefill_chunked", *ch(P, 8, 8, P, P, 9))                        # cap < min(NB, k+2)
    _expect(-2, "sparda_prefill_chunked", *ch(P, 8, 8, None, None, 0, T=4097 * 64))     # more than 4096 blocks
    _expect(-2, "sparda_prefill_chunked", *ch(P, 8, 8, None, None, 0, bs=32))           # two launches need the lists
    _expect(-2, "sparda_prefill_chunked", *ch(P, 8, 8, None, None, 0, Hq=13))           # Hq not a multiple of Hkv


def test_decode_workspace_size_formula():
    # the block scores of every (sequence, KV head), rounded up to 256 B
    up = lambda x: (x + 255) // 256 * 256
    B, S, Hq, Hkv, D, bs, k = 8, 16384, 12, 4, 64, 64, 8
    NB = S // bs
    want = up(B * Hkv * NB * 4)
    assert sparda.decode_workspace_bytes(B, S, Hq, Hkv, D, bs, k) == want


def test_dense_decode_split_workspace_size():
    # four blocks per split (more past 4096 splits per (sequence, KV head));
    # each split's partial is (m, l, o[D]) fp32 for each of the R heads
    lib = sparda.load()
    B, Hq, Hkv, D, bs = 1, 12, 4, 64, 64
    per_split = B * Hkv * (Hq // Hkv) * (D + 2) * 4
    assert lib.sparda_decode_dense_workspace_bytes(B, Hq, Hkv, D, 32768, bs) == 128 * per_split  # 512 blocks
    assert lib.sparda_decode_dense_workspace_bytes(B, Hq, Hkv, D, 8 * 64 + 1, bs) == 3 * per_split  # 9 blocks
    assert lib.sparda_decode_dense_workspace_bytes(B, Hq, Hkv, D, 4 * 64, bs) == 0  # one split: none
    assert lib.sparda_decode_dense_workspace_bytes(B, Hq, Hkv, D, 1 << 20, bs) == 4096 * per_split  # 16384 blocks
    assert lib.sparda_decode_dense_workspace_bytes(B, Hq, Hkv, D, 1 << 21, bs) == 4096 * per_split  # the cap


def test_offload_and_selected_decode_argument_errors():
    import ctypes
    P = 4096
    h = ctypes.c_void_p()
    _expect(-1, "sparda_offload_create", 1, 64, 4, 64, 1, None)
    _expect(-2, "sparda_offload_create", 1, 64, 4, 48, 1, ctypes.byref(h))  # D=48 unsupported
    _expect(-3, "sparda_offload_create", 1, 64, 4, 64, 5, ctypes.byref(h))
    _expect(-7, "sparda_offload_destroy", None)
    _expect(-7, "sparda_offload_append", None, P, P, 1, 1, 1, 0, 1, 64, None, None)
    _expect(-7, "sparda_offload_fetch", None, P, P, 10, 64, 100, 0, P, P, None)
    _expect(-1, "sparda_decode_selected", None, 1, 1, P, P, 8, 8, 8, 1, 0, None, None, 0, None, None, 0, 0,
            1, 100, 12, 4, 64, 64, 0.125, P, 1, None, 0, None)
    _expect(-6, "sparda_decode_selected", P, 1, 1, P, P, 8, 8, 8, 1, 1, None, None, 0, None, None, 0, 0,
            1, 100, 12, 4, 64, 64, 0.125, P, 1, None, 0, None)  # compact without a selection
    _expect(-2, "sparda_decode_selected", P, 1, 1, P, P, 8, 8, 8, 1, 0, P, P, 40, None, None, 0, 0,
            1, 100, 12, 4, 64, 64, 0.125, P, 1, None, 0, None)  # sel_cap > 34
    _expect(-5, "sparda_decode_selected", P, 1, 1, P + 2, P, 8, 8, 8, 1, 0, None, None, 0, None, None, 0, 0,
            1, 100, 12, 4, 64, 64, 0.125, P, 1, None, 0, None)  # misaligned K
    _expect(-4, "sparda_decode_selected", P, 1, 1, P, P, 8, 8, 8, 1, 0, None, None, 0, None, None, 0, 0,
            1, 100, 12, 4, 64, 64, 0.125, P, 1, P + 4, 4096, None)  # misaligned workspace
    _expect(-2, "sparda_select_decode", P, 1, 1, 1, P, 1, 4, 64, 64, 100, 50, 64, 8, 1, 0.125, P, P, 10,
            None)  # pos < len - 1
    _expect(-2, "sparda_select_decode", P, 1, 1, 1, P, 1, 4, 64, 64, 100, 100, 64, 8, 1, 0.125, P, P, 9,
            None)  # sel_cap < k + 2
    _expect(-6, "sparda_select_decode", P, 1, 1, 1, P, 1, 4, 64, 64, 100, 100, 64, 8, 3, 0.125, P, P, 10,
            None)  # unknown routing
    # teacher mass: q, q_sb, q_st, q_sh, k, k_sb, k_st, k_sh, dtype, B, T, Hq, Hkv, D, bs, causal, scale, mass, stream
    _expect(-1, "sparda_teacher_mass", None, 8, 8, 8, P, 8, 8, 8, 1, 1, 64, 12, 4, 64, 64, 1, 0.125, P, None)
    _expect(-3, "sparda_teacher_mass", P, 8, 8, 8, P, 8, 8, 8, 0, 1, 64, 12, 4, 64, 64, 1, 0.125, P, None)
    _expect(-2, "sparda_teacher_mass", P, 8, 8, 8, P, 8, 8, 8, 1, 1, 64, 12, 4, 64, 32, 1, 0.125, P, None)
    _expect(-2, "sparda_teacher_mass", P, 8, 8, 8, P, 8, 8, 8, 1, 1, 64, 16, 4, 64, 64, 1, 0.125, P, None)
    _expect(-5, "sparda_teacher_mass", P, 8, 4, 8, P, 8, 8, 8, 1, 1, 64, 12, 4, 64, 64, 1, 0.125, P, None)
    # fused producer: x, x_stride, w, M, C, Nq, Nk, Nf, eps, cos, sin, rope_len, T, pos0, q, k, v, f, f_dtype, stream
    _expect(-1, "sparda_produce", None, 768, P, 8, 768, 768, 256, 256, 1e-5, P, P, 64, 8, 0, P, P, P, P, 1, None)
    _expect(-3, "sparda_produce", P, 768, P, 8, 768, 768, 256, 256, 1e-5, P, P, 64, 8, 0, P, P, P, P, 7, None)
    _expect(-2, "sparda_produce", P, 768, P, 8, 768, 768, 256, 96, 1e-5, P, P, 64, 8, 0, P, P, P, P, 1, None)
    _expect(-2, "sparda_produce", P, 768, P, 8, 768, 768, 256, 256, 1e-5, P, P, 64, 8, 60, P, P, P, P, 1, None)
    _expect(-2, "sparda_produce", P, 768, P, 9, 768, 768, 256, 256, 1e-5, P, P, 64, 8, 0, P, P, P, P, 1, None)
    _expect(-5, "sparda_produce", P + 2, 768, P, 8, 768, 768, 256, 256, 1e-5, P, P, 64, 8, 0, P, P, P, P, 1, None)
    # block sums of a device cache: k, dtype, sb, st, sh, B, Hkv, D, pos, n, bs, nb_stride, sums, stream
    _expect(-1, "sparda_block_sums", None, 1, 256, 256, 64, 1, 4, 64, 0, 64, 64, 4, P, None)
    _expect(-3, "sparda_block_sums", P, 9, 256, 256, 64, 1, 4, 64, 0, 64, 64, 4, P, None)
    _expect(-2, "sparda_block_sums", P, 1, 256, 256, 64, 1, 4, 64, 0, 0, 64, 4, P, None)  # n = 0
    _expect(-8, "sparda_block_sums", P, 1, 256, 256, 64, 1, 4, 64, 200, 100, 64, 4, P, None)  # block 4 of 4
    _expect(-5, "sparda_block_sums", P, 1, -1, 256, 64, 1, 4, 64, 0, 64, 64, 4, P, None)


def test_device_position_entry_argument_errors():
    P = 4096
    Q = 4104  # 8-byte aligned position pointer; Q + 4 is not
    # produce_at: x, x_stride, w, M, C, Nq, Nk, Nf, eps, cos, sin, rope_len, T, pos_dev, q, k, v, f, f_dtype, stream
    _expect(-1, "sparda_produce_at", P, 768, P, 8, 768, 768, 256, 256, 1e-5, P, P, 64, 1, None, P, P, P, P, 1, None)
    _expect(-5, "sparda_produce_at", P, 768, P, 8, 768, 768, 256, 256, 1e-5, P, P, 64, 1, Q + 4, P, P, P, P, 1,
            None)
    _expect(-2, "sparda_produce_at", P, 768, P, 8, 768, 768, 256, 256, 1e-5, P, P, 64, 3, Q, P, P, P, P, 1,
            None)  # M not a multiple of T
    # append_at: kc, vc, dtype, sb, st, sh, k_new, v_new, new_sb, new_sh, B, Hkv, D, max_len, pos_dev, bs,
    #            nb_stride, sums, stream
    _expect(-1, "sparda_append_at", P, P, 1, 256, 256, 64, P, P, 256, 64, 1, 4, 64, 256, None, 64, 4, P, None)
    _expect(-1, "sparda_append_at", P, P, 1, 256, 256, 64, P, None, 256, 64, 1, 4, 64, 256, Q, 64, 4, P, None)
    _expect(-1, "sparda_append_at", P, None, 1, 256, 256, 64, P, P, 256, 64, 1, 4, 64, 256, Q, 64, 4, P, None)
    _expect(-8, "sparda_append_at", P, P, 1, 256, 256, 64, P, P, 256, 64, 1, 4, 64, 257, Q, 64, 4, P,
            None)  # 5 blocks > nb_stride 4
    _expect(-2, "sparda_append_at", P, P, 1, 256, 256, 64, P, P, 256, 64, 1, 4, 64, 0, Q, 64, 4, P, None)
    _expect(-3, "sparda_append_at", P, P, 5, 256, 256, 64, P, P, 256, 64, 1, 4, 64, 256, Q, 64, 4, P, None)
    # select_decode_at: f, f_dtype, f_sb, f_sh, sums, B, Hkv, D, nb_stride, max_len, pos_dev, bs, k, routing,
    #                   scale, sel, n_sel, sel_cap, lookahead, stream
    _expect(-1, "sparda_select_decode_at", P, 1, 1, 1, P, 1, 4, 64, 64, 100, None, 64, 8, 1, 0.125, P, P, 10, 0,
            None)
    _expect(-2, "sparda_select_decode_at", P, 1, 1, 1, P, 1, 4, 64, 1, 100, Q, 64, 8, 1, 0.125, P, P, 10, 0,
            None)  # nb_stride < ceil(max_len / bs)
    _expect(-2, "sparda_select_decode_at", P, 1, 1, 1, P, 1, 4, 64, 64, 100, Q, 64, 8, 1, 0.125, P, P, 9, 1,
            None)  # sel_cap < k + 2
    # decode_at: q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, compact, sel, n_sel, sel_cap, window_k,
    #            k_new, v_new, new_sb, new_sh, B, max_len, pos_dev, Hq, Hkv, D, bs, scale, out, out_sb, stream
    _expect(-1, "sparda_decode_at", P, 1, 1, P, P, 8, 8, 8, 1, 0, None, None, 0, 8, None, None, 0, 0, 1, 100, None,
            12, 4, 64, 64, 0.125, P, 1, None, 0, None)
    _expect(-6, "sparda_decode_at", P, 1, 1, P, P, 8, 8, 8, 1, 0, P, P, 10, 8, None, None, 0, 0, 1, 100, Q, 12, 4,
            64, 64, 0.125, P, 1, None, 0, None)  # a list and a window
    _expect(-6, "sparda_decode_at", P, 1, 1, P, P, 8, 8, 8, 1, 1, None, None, 0, 8, None, None, 0, 0, 1, 100, Q,
            12, 4, 64, 64, 0.125, P, 1, None, 0, None)  # compact buffers without a selection
    _expect(-1, "sparda_decode_at", P, 1, 1, P, P, 8, 8, 8, 1, 0, P, P, 10, 0, P, None, 8, 8, 1, 100, Q, 12, 4,
            64, 64, 0.125, P, 1, None, 0, None)  # k_new without v_new
    _expect(-2, "sparda_decode_at", P, 1, 1, P, P, 8, 8, 8, 1, 0, None, None, 0, 33, None, None, 0, 0, 1, 100, Q,
            12, 4, 64, 64, 0.125, P, 1, None, 0, None)  # window > 32
    _expect(-5, "sparda_decode_at", P, 1, 1, P + 2, P, 8, 8, 8, 1, 0, None, None, 0, 8, None, None, 0, 0, 1, 100,
            Q, 12, 4, 64, 64, 0.125, P, 1, None, 0, None)  # misaligned K
    # offload entries at a device position (handle checks come first)
    _expect(-7, "sparda_offload_fetch_at", None, P, P, 10, 64, Q, P, P, None)
    _expect(-7, "sparda_offload_append_at", None, P, P, 256, 64, Q, 64, P, None)


def test_ffn_decode_argument_errors():
    P = 4096
    # x, x_stride, w_gate_up, w_down, M, C, F, eps, act, out, out_stride, stream
    _expect(-1, "sparda_ffn_decode", None, 768, P, P, 1, 768, 2048, 1e-5, P, P, 768, None)
    _expect(-2, "sparda_ffn_decode", P, 768, P, P, 17, 768, 2048, 1e-5, P, P, 768, None)   # 17 rows
    _expect(-2, "sparda_ffn_decode", P, 768, P, P, 1, 800, 2048, 1e-5, P, P, 800, None)    # C % 128
    _expect(-2, "sparda_ffn_decode", P, 768, P, P, 1, 768, 4096, 1e-5, P, P, 768, None)    # F > 2048
    _expect(-5, "sparda_ffn_decode", P + 2, 768, P, P, 1, 768, 2048, 1e-5, P, P, 768, None)


def test_decode_sums_argument_errors():
    P = 4096
    # q, q_sb, q_sh, k, v, kv_sb, kv_ss, kv_sh, dtype, f, f_dtype, f_sb, f_sh, sums, nb_stride, update, B, S, pos_dev,
    # Hq, Hkv, D, bs, top_k, routing, scale, route_scale, sel_out, n_sel_out, out, out_sb, stream
    _expect(-1, "sparda_decode_sums", P, 1, 1, P, P, 8, 8, 8, 1, None, 1, 1, 1, P, 64, 0, 1, 100, None, 12, 4, 64, 64,
            8, 1, 0.125, 0.125, None, None, P, 1, None)
    _expect(-6, "sparda_decode_sums", P, 1, 1, P, P, 8, 8, 8, 1, P, 1, 1, 1, P, 64, 0, 1, 100, None, 12, 4, 64, 64,
            8, 5, 0.125, 0.125, None, None, P, 1, None)  # unknown routing
    _expect(-2, "sparda_decode_sums", P, 1, 1, P, P, 8, 8, 8, 1, P, 1, 1, 1, P, 1, 0, 1, 100, None, 12, 4, 64, 64,
            8, 1, 0.125, 0.125, None, None, P, 1, None)  # nb_stride < ceil(S / bs)
    _expect(-2, "sparda_decode_sums", P, 1, 1, P, P, 8, 8, 8, 1, P, 1, 1, 1, P, 64, 0, 1, 100, None, 12, 4, 64, 64,
            40, 1, 0.125, 0.125, None, None, P, 1, None)  # top_k > 32
    _expect(-5, "sparda_decode_sums", P, 1, 1, P, P, 8, 8, 8, 1, P, 1, 1, 1, P + 4, 64, 0, 1, 100, None, 12, 4, 64,
            64, 8, 1, 0.125, 0.125, None, None, P, 1, None)  # misaligned block sums
