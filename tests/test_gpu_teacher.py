"""GPU parity of the teacher block mass kernel (TeacherBlockSelector steps 1-3,
model/forecast.py:141-193, from q and k) against the float64 oracle; masses are
probabilities, compared within max-abs 1e-4 (fp32 bar)."""

import numpy as np
import pytest
import torch

import sparda
from model.forecast import TeacherBlockSelector
from oracle import sparda_oracle as O
from helpers import np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("B,T,Hq,Hkv,causal", [(2, 333, 12, 4, True), (1, 1024, 12, 4, True),
                                               (2, 200, 12, 4, False), (1, 130, 4, 4, True),
                                               (1, 257, 4, 2, False)])
def test_teacher_mass_matches_oracle(B, T, Hq, Hkv, causal):
    case(f"teacher mass B={B} T={T} Hq={Hq} Hkv={Hkv} causal={causal}")
    g = torch.Generator().manual_seed(T + Hq)
    q = torch.randn(B, T, Hq, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(B, T, Hkv, 64, generator=g).to(torch.bfloat16)
    got = sparda.teacher_block_mass(q.to(DEV), k.to(DEV), 64, causal=causal)
    want = O.teacher_block_mass(np32(q), np32(k), 64, causal)
    assert got.shape == want.shape
    err = np.abs(got.cpu().numpy() - want)
    assert err.max() < 1e-4, err.max()
    if causal:
        nb = want.shape[-1]
        future = np.arange(nb)[None, :] > (np.arange(T) // 64)[:, None]
        assert (got.cpu().numpy()[..., future] == 0).all()


def test_teacher_selector_from_qk_matches_materialised_weights():
    case("TeacherBlockSelector.from_qk vs forward on dense weights")
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 512, 12, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 512, 4, 64, generator=g).to(torch.bfloat16)
    sel = TeacherBlockSelector(block_size=64, num_queries_per_kv=3)
    s_k, tk_k, tg_k = sel.from_qk(q.to(DEV), k.to(DEV), top_k=4)
    w = torch.from_numpy(O.dense_weights(np32(q), np32(k)))
    s_r, tk_r, tg_r = sel(w, top_k=4)
    assert np.abs(s_k.cpu().numpy() - s_r.numpy()).max() < 1e-4
    assert np.abs(tg_k.cpu().numpy() - tg_r.numpy()).max() < 1e-4
    # top-k equal wherever the 4th and 5th teacher scores are apart
    srt = np.sort(s_r.numpy(), axis=-1)[..., ::-1]
    clear = (srt[..., 3] - srt[..., 4]) > 1e-3
    assert (tk_k.cpu().numpy()[clear] == tk_r.numpy()[clear]).all()
