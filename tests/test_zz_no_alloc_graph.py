"""mlxr_qgemm_run_noalloc captured in a HIP graph, its stated purpose: a split-K call
(M = 512, N = K = 4096: the tiled launch splits K into the library's scratch array) captured
once and replayed, with eager work and synchronisations between replays, equals the eager
call bit for bit on every replay.  It runs in a fresh process so that the capture holds the
process's first no-alloc call: the per-device scratch address is looked up inside it."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
import mlxr_amd as mx
from mlxr_amd import qgemm

dev = torch.device("cuda:0")
Q4K, N, K, M = 3, 4096, 4096, 512
need = mx.workspace_size(Q4K, N, K, M)
assert need > 0, need  # the call splits K
pw = mx.pack_weights(mx.synth_gguf(Q4K, N, K, 21), N, K, Q4K, device=dev)
bits = mx.synth_act(M * K, mx.BF16, 22)
x = torch.from_numpy(bits.view(np.int16).reshape(M, K)).to(dev).view(torch.bfloat16)
y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
lib = qgemm.lib()

def call(stream):
    rc = lib.mlxr_qgemm_run_noalloc(Q4K, N, K, 0, pw.data_ptr(), x.data_ptr(), mx.BF16, None, mx.F32,
                                    y.data_ptr(), mx.BF16, M, 0, stream)
    assert rc == 0, lib.mlxr_qgemm_last_error()

s = torch.cuda.Stream()
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    call(s.cuda_stream)  # the process's first no-alloc call
torch.cuda.synchronize()
# eager reference through the workspace entry point (the same plan, the same kernels)
ws = torch.empty(need, dtype=torch.uint8, device=dev)
ref = torch.empty_like(y)
rc = lib.mlxr_qgemm_run_ws(Q4K, N, K, 0, pw.data_ptr(), x.data_ptr(), mx.BF16, None, mx.F32, ref.data_ptr(),
                           mx.BF16, M, 0, ws.data_ptr(), need, None)
assert rc == 0, lib.mlxr_qgemm_last_error()
torch.cuda.synchronize()
for rep in range(3):
    y.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref), rep
    call(None)  # eager work between replays, on the same scratch array
    torch.cuda.synchronize()
    assert torch.equal(y, ref), rep
print("ok")
"""


def test_noalloc_graph_capture_replays(cuda):
    r = subprocess.run([sys.executable, "-c", SCRIPT, ROOT], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-2000:] + r.stderr[-2000:]
