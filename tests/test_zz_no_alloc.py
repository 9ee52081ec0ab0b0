"""omni_lmhead_argmax_noalloc (lm_head + greedy argmax with library-held candidate slots)
against the allocating pair omni_lmhead_candidates + omni_argmax_finalize (candidates in
caller buffers), through the C ABI: two calls in a row, the second with a smaller input,
ids / logits / next_ids / lengths bit-equal; shapes the entry point does not take rejected
before any launch; and, in a fresh process, the entry point's very first call made inside
a HIP graph capture (the callers it is for), the graph replayed against the allocating
pair with eager work between the replays."""

import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

H = 1536


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def _case(gpu, M, V, seed):
    from omniserver_amd.linear import LMHeadArgmax
    g = torch.Generator().manual_seed(seed)
    E = (torch.randn(V, H, generator=g) * 0.02).half()
    h = torch.randn(M, H, generator=g).half()
    E[7] = E[3]                          # two equal columns: ties resolve to the lower index
    return LMHeadArgmax(E.to(gpu)), h.to(gpu)


def _noalloc(lm, h, M, V, logits, ids, nxt, lens):
    from omniserver_amd._lib import lib, ptr, stream
    return lib().omni_lmhead_argmax_noalloc(ptr(h), h.stride(0), ptr(lm.table_packed), M, V, H,
                                            ptr(logits), ptr(ids), ptr(nxt), ptr(lens), stream())


def test_noalloc_lmhead_argmax_matches_allocating_path(gpu):
    for M, V, seed in ((33, 151936, 1), (5, 32768, 2)):      # the second call is smaller
        say(f"no-alloc lm_head argmax M={M} V={V}")
        lm, h = _case(gpu, M, V, seed)
        ids_ref = torch.empty(M, dtype=torch.int64, device=gpu)
        logits_ref = torch.empty(M, V, dtype=torch.float16, device=gpu)
        lm.argmax_out(h, ids_ref, logits_ref)
        ids = torch.full((M,), -1, dtype=torch.int64, device=gpu)
        nxt = torch.full((M,), -1, dtype=torch.int64, device=gpu)
        lens = torch.arange(M, dtype=torch.int64, device=gpu) * 3
        logits = torch.empty(M, V, dtype=torch.float16, device=gpu)
        assert _noalloc(lm, h, M, V, logits, ids, nxt, lens) == 0
        torch.cuda.synchronize()
        assert torch.equal(ids.cpu(), ids_ref.cpu())
        assert torch.equal(logits.cpu(), logits_ref.cpu())
        assert torch.equal(nxt.cpu(), ids.cpu())
        assert torch.equal(lens.cpu(), torch.arange(M, dtype=torch.int64) * 3 + 1)
        assert torch.equal(ids.cpu(), logits.float().cpu().argmax(-1))     # first max
        # without the optional outputs
        ids2 = torch.full((M,), -1, dtype=torch.int64, device=gpu)
        assert _noalloc(lm, h, M, V, None, ids2, None, None) == 0
        torch.cuda.synchronize()
        assert torch.equal(ids2.cpu(), ids_ref.cpu())


def test_noalloc_lmhead_argmax_rejects_unsupported_shapes(gpu):
    """More than 64 rows, a vocabulary that is not whole 32-column tiles, and a missing ids
    output are refused before anything is launched (real, small device buffers are passed,
    so a launch would not run on a wild pointer either).  The library's array holds the
    candidates of grids up to 512 workgroups; the grid is one workgroup per CU, so that
    bound cannot be reached on this part and is not exercised here."""
    from omniserver_amd._lib import lib, ptr, stream
    say("no-alloc lm_head argmax: shapes it does not take")
    L = lib()
    x = torch.zeros(65, H, dtype=torch.float16, device=gpu)
    table = torch.zeros(32768 * H, dtype=torch.float16, device=gpu)
    ids = torch.zeros(65, dtype=torch.int64, device=gpu)
    assert L.omni_lmhead_argmax_noalloc(ptr(x), H, ptr(table), 65, 32768, H, None, ptr(ids),
                                        None, None, stream()) == -2
    assert L.omni_lmhead_argmax_noalloc(ptr(x), H, ptr(table), 4, 32760, H, None, ptr(ids),
                                        None, None, stream()) == -2
    assert L.omni_lmhead_argmax_noalloc(ptr(x), H, ptr(table), 4, 32768, H, None, None, None,
                                        None, stream()) == -1
    torch.cuda.synchronize()
    assert int(ids.abs().sum()) == 0       # nothing was written


_CAPTURE_CHILD = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from omniserver_amd._lib import lib, ptr, stream
from omniserver_amd.linear import LMHeadArgmax
H, V, M = 1536, 151936, 12
dev = torch.device("cuda:0")
g = torch.Generator().manual_seed(9)
lm = LMHeadArgmax((torch.randn(V, H, generator=g) * 0.02).half().to(dev))
h = torch.randn(M, H, generator=g).half().to(dev)
ids = torch.full((M,), -1, dtype=torch.int64, device=dev)
logits = torch.empty(M, V, dtype=torch.float16, device=dev)
ids_ref = torch.empty(M, dtype=torch.int64, device=dev)
logits_ref = torch.empty(M, V, dtype=torch.float16, device=dev)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
rc = []
with torch.cuda.graph(graph):                 # the entry point's first call in this process
    rc.append(lib().omni_lmhead_argmax_noalloc(ptr(h), H, ptr(lm.table_packed), M, V, H,
                                               ptr(logits), ptr(ids), None, None, stream()))
assert rc == [0], rc
for rep in range(4):
    h.copy_(torch.randn(M, H, generator=g).half())     # eager work between the replays
    ids.fill_(-1)
    graph.replay()
    lm.argmax_out(h, ids_ref, logits_ref)             # the allocating pair, eagerly
    torch.cuda.synchronize()
    assert torch.equal(ids.cpu(), ids_ref.cpu()), rep
    assert torch.equal(logits.cpu(), logits_ref.cpu()), rep
print("capture-first-call ok", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(gpu):
    say("no-alloc lm_head argmax: first call inside a graph capture (fresh process)")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True,
                         text=True, timeout=180)
    say(res.stdout.strip()[-400:])
    assert res.returncode == 0, res.stderr[-2000:]
    assert "capture-first-call ok" in res.stdout
