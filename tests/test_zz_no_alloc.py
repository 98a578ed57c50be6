"""ccinfer_decode_attention_noalloc (static per-GPU scratch, no workspace, no allocation)
against ccinfer_decode_attention with a caller workspace: bit-identical outputs on two calls
in a row, the second with a smaller batch, plus a shape whose scratch need exceeds the
static array, which is rejected."""
import ctypes

import pytest
import torch

from ccinfer_amd import _lib
from ccinfer_amd import workloads as W
from tests._util import say

pytestmark = pytest.mark.gpu

INVALID = 6


def _with_workspace(lib, w, meta, out, stream):
    n = lib.ccinfer_decode_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d, 16)
    ws = torch.zeros(max(1, n), dtype=torch.uint8, device=w.q.device)
    rc = lib.ccinfer_decode_attention(
        w.q.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
        meta["block_table"].data_ptr(), meta["context_lens"].data_ptr(), out.data_ptr(),
        w.batch, w.mbpr, w.hq, w.hkv, w.d, 16, ws.data_ptr(), n, stream)
    assert rc == 0, rc
    return n


def _no_alloc(lib, w, meta, out, stream):
    return lib.ccinfer_decode_attention_noalloc(
        w.q.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
        meta["block_table"].data_ptr(), meta["context_lens"].data_ptr(), out.data_ptr(),
        w.batch, w.mbpr, w.hq, w.hkv, w.d, 16, stream)


def test_no_alloc_decode_matches_workspace_decode(gpu):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    # configs[4] shape (split-KV, balanced plan), then a smaller configs[1]-like batch
    cases = [("decode b32 ctx32768 gqa4", W.decode_long(device=gpu, seed=51)),
             ("decode b16 ctx U[128,2048]",
              W.decode_batched(device=gpu, seed=52, batch=16, ctx_hi=2048, with_write=False))]
    for name, w in cases:
        say(f"no-alloc {name}")
        meta = w.device_meta(gpu)
        want = torch.full_like(w.q, float("nan"))
        got = torch.full_like(w.q, float("nan"))
        need = _with_workspace(lib, w, meta, want, stream)
        assert need > 0  # exercises the static scratch
        assert _no_alloc(lib, w, meta, got, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), name


def test_no_alloc_rejects_shapes_beyond_the_static_scratch(gpu):
    say("no-alloc rejects a shape needing more than 32 MiB of scratch")
    lib = _lib.load()
    b, mbpr, hq, hkv, d = 256, 2048, 32, 8, 128
    assert lib.ccinfer_decode_workspace_size(b, mbpr, hq, hkv, d, 16) > (32 << 20)
    fake = ctypes.c_void_p(0x1000)
    assert lib.ccinfer_decode_attention_noalloc(fake, fake, fake, fake, fake, fake, b, mbpr, hq,
                                                hkv, d, 16, None) == INVALID


def test_no_alloc_decode_under_graph_capture(gpu):
    """The entry's intended caller: a decode captured in a HIP graph without a workspace.
    Each replay (with eager work and synchronisations between) equals the eager call."""
    say("no-alloc decode captured in a graph")
    lib = _lib.load()
    w = W.decode_batched(device=gpu, seed=53, batch=40, ctx_hi=3000, with_write=False)
    meta = w.device_meta(gpu)
    out = torch.full_like(w.q, float("nan"))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert _no_alloc(lib, w, meta, out, s.cuda_stream) == 0
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        rc = _no_alloc(lib, w, meta, out, s.cuda_stream)
    assert rc == 0
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep


_FIRST_CALL_IN_CAPTURE = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from ccinfer_amd import _lib
from ccinfer_amd import workloads as W
from tests.test_zz_no_alloc import _no_alloc, _with_workspace
dev = torch.device("cuda:0")
lib = _lib.load()
w = W.decode_batched(device=dev, seed=54, batch=24, ctx_hi=2500, with_write=False)
meta = w.device_meta(dev)
out = torch.full_like(w.q, float("nan"))
want = torch.full_like(w.q, float("nan"))
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):
    rc = _no_alloc(lib, w, meta, out, s.cuda_stream)   # the process's first no-alloc call
assert rc == 0, rc
_with_workspace(lib, w, meta, want, torch.cuda.current_stream().cuda_stream)
torch.cuda.synchronize()
for rep in range(3):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), rep
print("ok")
"""


def test_no_alloc_first_call_under_capture(gpu):
    """The scratch address is resolved by the first call; here that call is made while the
    stream is being captured, in a fresh process (so nothing resolved it earlier)."""
    import subprocess
    import sys
    from pathlib import Path
    say("no-alloc first call inside graph capture (fresh process)")
    root = str(Path(__file__).resolve().parent.parent)
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root],
                         capture_output=True, text=True, timeout=150, cwd=root)
    assert res.returncode == 0 and "ok" in res.stdout, res.stdout[-2000:] + res.stderr[-2000:]
