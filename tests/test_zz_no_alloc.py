"""The allocation-free decode entry point (sparda_decode_noalloc) against the
workspace one (sparda_decode), called through the C ABI: same inputs, same
kernels, so outputs, selections and prototypes must be identical. Two calls in
a row, the second smaller, both share the library's scratch array."""

import ctypes
import os
import sys

import pytest
import torch

import sparda
from sparda import _lib, synth
from oracle import sparda_oracle as O
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _run(entry, x, S, bs, k, routing, ws=None):
    q, kc, vc, f = x["q"], x["k_cache"], x["v_cache"], x["forecast"]
    B, Hq, D = q.shape
    Hkv = kc.shape[2]
    NB = (S + bs - 1) // bs
    out = torch.full((B, Hq * D), float("nan"), dtype=q.dtype, device=DEV)
    protos = torch.full((B, NB, Hkv, D), float("nan"), dtype=torch.float32, device=DEV)
    sel = torch.full((B, Hkv, k + 2), -7, dtype=torch.int32, device=DEV)
    n_sel = torch.full((B, Hkv), -7, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    args = [q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), _lib.BF16, f.data_ptr(), _lib.BF16, f.stride(0), f.stride(1), B, S, Hq, Hkv, D, bs, k,
            routing, float(D) ** -0.5, None, protos.data_ptr(), sel.data_ptr(), n_sel.data_ptr(),
            out.data_ptr(), out.stride(0)]
    if entry == "sparda_decode":
        args += [ws.data_ptr(), ws.numel()]
    _lib.call(entry, *args, stream)
    torch.cuda.synchronize()
    return out, protos, sel, n_sel


@pytest.mark.parametrize("routing", [_lib.ROUTE_ABSOLUTE, _lib.ROUTE_REFERENCE])
def test_noalloc_decode_equals_workspace_decode_twice(routing):
    bs, k = 64, 8
    # the decode workload (B=8, 16K cache), then a smaller, ragged step
    for B, S, seed in ((8, 16384, 1002), (3, 5000, 77)):
        print(f"[case] decode_noalloc B={B} S={S} routing={routing}", flush=True)
        x = {n: t.to(DEV) for n, t in synth.decode_inputs(B, S, 12, 4, 64, dtype=torch.bfloat16,
                                                            seed=seed).items()}
        nbytes = sparda.decode_workspace_bytes(B, S, 12, 4, 64, bs, k)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        want = _run("sparda_decode", x, S, bs, k, routing, ws)
        got = _run("sparda_decode_noalloc", x, S, bs, k, routing)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        # and the oracle agrees on the attention output
        rmode = "absolute" if routing == _lib.ROUTE_ABSOLUTE else "reference"
        kc = np32(x["k_cache"])
        sel_o, n_o, _ = O.decode_selection(kc, S, np32(x["forecast"]), bs, k, rmode)
        assert (got[3].cpu().numpy() == n_o).all() and (got[2].cpu().numpy() == sel_o).all()
        ref = O.attention_decode(np32(x["q"]), kc, np32(x["v_cache"]), S, sel_o, n_o, bs)
        assert_close_out(np32(got[0]), ref, torch.bfloat16)


def test_noalloc_decode_rejects_steps_beyond_its_scratch():
    # 64 x 8 heads x 1024 blocks = 524,288 scores > the 262,144 the scratch holds;
    # rejected before any launch (pointers are never dereferenced)
    P = 4096
    with pytest.raises(sparda.SpardaArgumentError) as ei:
        _lib.call("sparda_decode_noalloc", P, 64, 64, P, P, 8 * 65536 * 64, 8 * 64, 64, _lib.BF16, P, _lib.BF16,
                  512, 64, 64, 65536, 8, 8, 64, 64, 8, _lib.ROUTE_ABSOLUTE, 0.125, None, None, None, None, P,
                  512, None)
    assert ei.value.code == -8


# Run in a fresh process, so that the library's first noalloc call on the
# device (the one that looks up the scratch array's address) happens while the
# stream is being captured into a HIP graph; the graph is then replayed with
# eager work between the replays, each replay checked against the workspace
# entry point's eager result.
_CAPTURE_SCRIPT = r"""
import sys
sys.path[:0] = sys.argv[1:4]
import torch
import sparda
from sparda import _lib, synth
from test_zz_no_alloc import _run

DEV = "cuda"
B, S, bs, k = 4, 4096 + 37, 64, 8
x = {n: t.to(DEV) for n, t in synth.decode_inputs(B, S, 12, 4, 64, dtype=torch.bfloat16, seed=91).items()}
ws = torch.empty(sparda.decode_workspace_bytes(B, S, 12, 4, 64, bs, k), dtype=torch.uint8, device=DEV)
want = _run("sparda_decode", x, S, bs, k, _lib.ROUTE_ABSOLUTE, ws)
q, kc, vc, f = x["q"], x["k_cache"], x["v_cache"], x["forecast"]
NB = (S + bs - 1) // bs
out = torch.full((B, 12 * 64), float("nan"), dtype=q.dtype, device=DEV)
protos = torch.full((B, NB, 4, 64), float("nan"), dtype=torch.float32, device=DEV)
sel = torch.full((B, 4, k + 2), -7, dtype=torch.int32, device=DEV)
n_sel = torch.full((B, 4), -7, dtype=torch.int32, device=DEV)
side = torch.cuda.Stream()
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
print("[capture] first sparda_decode_noalloc call of the process, under capture", flush=True)
with torch.cuda.graph(g, stream=side):
    _lib.call("sparda_decode_noalloc", q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
              kc.stride(0), kc.stride(1), kc.stride(2), _lib.BF16, f.data_ptr(), _lib.BF16, f.stride(0),
              f.stride(1), B, S, 12, 4, 64, bs, k, _lib.ROUTE_ABSOLUTE, 0.125, None, protos.data_ptr(),
              sel.data_ptr(), n_sel.data_ptr(), out.data_ptr(), out.stride(0), side.cuda_stream)
for rep in range(3):
    for t in (out, protos):
        t.fill_(float("nan"))
    sel.fill_(-7)
    n_sel.fill_(-7)
    g.replay()
    torch.cuda.synchronize()
    for a, b in zip((out, protos, sel, n_sel), want):
        assert torch.equal(a, b), f"replay {rep} differs from the workspace entry point"
    # eager work on the device between the replays
    _run("sparda_decode", x, S, bs, k, _lib.ROUTE_ABSOLUTE, ws)
print("[capture] ok: 3 replays equal the workspace entry point", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    import subprocess
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    pkg = os.path.join(root, "local-research-small-language-model_amd")
    print("[case] decode_noalloc: first call of a fresh process under graph capture, 3 replays", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, root, pkg, here], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-2000:], r.stderr[-4000:], flush=True)
    assert r.returncode == 0, f"capture subprocess exited {r.returncode}"
    assert "[capture] ok" in r.stdout
