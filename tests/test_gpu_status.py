"""The device status word (sparda_status): zero after ordinary launches; raised,
together with NaN windows, when the compacted prefill abandons ordering waits.
The abandoned waits are forced from the host (SPARDA_PREFILL_WAIT_LIMIT=0: a
wait not ready at its first poll is given up) in a fresh process; every wave
still runs to completion."""

import json
import os
import subprocess
import sys

import pytest
import torch

import sparda
from sparda import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_status_word_is_clear_after_ordinary_launches():
    print("[case] status word after routed and list prefills", flush=True)
    sparda.status()  # clear whatever earlier tests left
    x = {n: t.to(DEV) for n, t in synth.prefill_inputs(4, 4096, 12, 4, 64, dtype=torch.bfloat16, seed=1001).items()}
    protos = sparda.compress(x["k"], 64)
    out, sel, n = sparda.prefill_routed(x["q"], x["k"], x["v"], x["forecast"], protos, 64, 8, want_sel=True)
    out2 = sparda.prefill(x["q"], x["k"], x["v"], sel, n, 64)
    assert torch.isfinite(out.float()).all() and torch.isfinite(out2.float()).all()
    assert sparda.status() == 0
    assert sparda.status(clear=False) == 0


_FORCED = r"""
import json, sys
sys.path[:0] = sys.argv[1:3]
import torch
import sparda
from sparda import synth
x = {n: t.to("cuda") for n, t in synth.prefill_inputs(4, 4096, 12, 4, 64, dtype=torch.bfloat16, seed=1001).items()}
protos = sparda.compress(x["k"], 64)
_, _, sel, n = sparda.route(x["forecast"], protos, 64, 8, want_topk=False, want_sel=True)
res = []
for _ in range(3):
    sparda.status()
    out = sparda.prefill(x["q"], x["k"], x["v"], sel, n, 64)
    word = sparda.status(clear=False)
    nan = torch.isnan(out.float()).view(4, 32, 128, 4, 3 * 64)  # (b, window, token, KV head group, cols)
    whole = nan.all(dim=-1).all(dim=2)  # windows whose group rows are NaN throughout
    part = nan.any(dim=-1).any(dim=2)
    res.append({"word": word, "nan_windows": int(whole.sum()), "partly_nan": int((part & ~whole).sum()),
                "finite_elsewhere": bool(torch.isfinite(out.float().view(4, 32, 128, 4, 192)[~part[:, :, None, :, None]
                                                                                  .expand(-1, -1, 128, -1, 192)]).all())})
    print("[forced] launch", res[-1], flush=True)
print("RESULT " + json.dumps(res), flush=True)
"""


def test_abandoned_waits_set_the_status_word_and_poison_whole_windows():
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    pkg = os.path.join(root, "local-research-small-language-model_amd")
    print("[case] forced wait timeouts (SPARDA_PREFILL_WAIT_LIMIT=0), B=4 T=4096, fresh process", flush=True)
    env = dict(os.environ, SPARDA_PREFILL_WAIT_LIMIT="0")
    r = subprocess.run([sys.executable, "-c", _FORCED, root, pkg], capture_output=True, text=True, timeout=300,
                       env=env)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0
    res = json.loads([ln for ln in r.stdout.splitlines() if ln.startswith("RESULT ")][-1][len("RESULT "):])
    for launch in res:
        # flagged exactly when some window was poisoned; poisoning covers whole
        # (window, KV head group) blocks and leaves every other row finite
        assert (launch["word"] & sparda.STATUS_PREFILL_WAIT_TIMEOUT != 0) == (launch["nan_windows"] > 0)
        assert launch["partly_nan"] == 0 and launch["finite_elsewhere"]
    assert any(launch["nan_windows"] > 0 for launch in res), "no wait was abandoned in three launches"
