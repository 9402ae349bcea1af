"""The reference's debug switches, each read once when the library loads, so
every case runs in a child process with the variable set:

* PYTORCH_NO_SUPA_MEMORY_CACHING (SUPACachingAllocator.cpp:2975-2978): no
  caching -- a freed tensor's device memory goes straight back to hipFree,
  so the allocator's reserved bytes fall back when a tensor dies;
* SUPA_LAUNCH_BLOCKING / CUDA_LAUNCH_BLOCKING (SUPAMiscFunctions.cpp:10-12):
  each launch is followed by a synchronisation, so an nll_loss target out of
  range raises IndexError at the nll_loss call itself (without the switch it
  surfaces at the next synchronize; tests/test_gpu_ops.py covers that).

Results stay correct in both modes."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PRELUDE = """
import sys
import torch
import torch_supa
import torch.nn.functional as F
torch.supa.set_cpu_fallback_enabled(False)
"""

UNCACHED = PRELUDE + """
x = torch.randn(1000, 1000)
d = x.to("supa")
torch.supa.synchronize()
r0 = torch.supa.memory_stats()["reserved_bytes"]
y = d * 2 + 1
torch.supa.synchronize()
r1 = torch.supa.memory_stats()["reserved_bytes"]
assert torch.equal(y.cpu(), x * 2 + 1)
del y
torch.supa.synchronize()
r2 = torch.supa.memory_stats()["reserved_bytes"]
assert r1 > r0 and r2 == r0, (r0, r1, r2)
print("OK", r0, r1, r2)
"""

BLOCKING = PRELUDE + """
logits = torch.randn(8, 10)
lp = F.log_softmax(logits.to("supa"), dim=1)
good = torch.tensor([1, 2, 3, 4, 5, 6, 7, 8])
assert torch.allclose(F.nll_loss(lp, good.to("supa")).cpu(), F.nll_loss(F.log_softmax(logits, 1), good), rtol=1e-5)
bad = good.clone()
bad[7] = 11
try:
    F.nll_loss(lp, bad.to("supa"))
except IndexError:
    pass
else:
    print("nll_loss with an out-of-range target did not raise at the call")
    sys.exit(1)
x = torch.randn(4096)
assert torch.equal((x.to("supa") + 1).cpu(), x + 1)
print("OK")
"""


def _run(script, **env_extra):
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([os.path.join(ROOT, "torch-supa_amd"), ROOT]), **env_extra)
    print("child process with", env_extra, flush=True)
    r = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "OK" in r.stdout, r.stdout + r.stderr


def test_no_memory_caching():
    _run(UNCACHED, PYTORCH_NO_SUPA_MEMORY_CACHING="1")


@pytest.mark.parametrize("var", ["SUPA_LAUNCH_BLOCKING", "CUDA_LAUNCH_BLOCKING"])
def test_launch_blocking_reports_at_the_launch(var):
    _run(BLOCKING, **{var: "1"})
