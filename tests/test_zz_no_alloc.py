"""rv_rmsnorm_bwd_noalloc (the RMSNorm backward that allocates nothing, its
dweight partials in a static device array) against rv_rmsnorm_bwd (caller
workspace), through the C ABI: bit-identical dx and dw on two calls in a row,
the second with a smaller input, so the second call runs over the first
call's leftover scratch contents."""
from __future__ import annotations

import ctypes
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest
import torch

from reversability_amd import _hip

EPS = float(torch.finfo(torch.float32).eps)


def _inputs(rows, width, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, width, generator=g)
    w = 1 + 0.02 * torch.randn(width, generator=g)
    dy = torch.randn(rows, width, generator=g)
    x, w, dy = x.to(dev), w.to(dev), dy.to(dev)
    _, rstd = _hip.ops.rmsnorm_fwd(x, w, EPS)
    return x, w, dy, rstd


def _with_workspace(lib, x, w, dy, rstd):
    rows, width = x.shape
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    nbytes = lib.rv_rmsnorm_bwd_workspace_bytes(rows, width)
    ws = torch.empty(nbytes // 4, device=x.device)
    st = lib.rv_rmsnorm_bwd(x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(),
                            dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), nbytes, rows, width,
                            _hip._stream(x))
    assert st == 0, lib.rv_status_string(st)
    return dx, dw


def _noalloc(lib, x, w, dy, rstd):
    rows, width = x.shape
    dx = torch.full_like(x, float("nan"))
    dw = torch.full_like(w, float("nan"))
    st = lib.rv_rmsnorm_bwd_noalloc(x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(),
                                    dx.data_ptr(), dw.data_ptr(), rows, width, _hip._stream(x))
    assert st == 0, lib.rv_status_string(st)
    return dx, dw


@pytest.mark.gpu
@pytest.mark.parametrize("shapes", [
    ((14848, 256), (1000, 256)),    # configs[0], then fewer rows
    ((32768, 1024), (4099, 1020)),  # configs[4]'s norm width, then a narrower ragged one
    ((300, 4096), (7, 66)),         # the maximum width, then the scalar path
    ((100000, 256), (40000, 256)),  # 782 then 313 partial rows: the batched reduce
])
def test_noalloc_matches_workspace_entry_point(cuda_device, shapes):
    lib = _hip.library()
    for i, (rows, width) in enumerate(shapes):
        print(f"[noalloc] call {i}: rows={rows} width={width}", flush=True)
        x, w, dy, rstd = _inputs(rows, width, 1337 + i, cuda_device)
        ref_dx, ref_dw = _with_workspace(lib, x, w, dy, rstd)
        dx, dw = _noalloc(lib, x, w, dy, rstd)
        torch.cuda.synchronize()
        assert torch.equal(dx, ref_dx), (rows, width)
        assert torch.equal(dw, ref_dw), (rows, width)


@pytest.mark.gpu
def test_noalloc_rejects_sizes_beyond_its_scratch(cuda_device):
    lib = _hip.library()
    x = torch.zeros(4, 8192, device=cuda_device)
    w = torch.ones(8192, device=cuda_device)
    rstd = torch.ones(4, device=cuda_device)
    st = lib.rv_rmsnorm_bwd_noalloc(x.data_ptr(), w.data_ptr(), x.data_ptr(), rstd.data_ptr(),
                                    x.data_ptr(), w.data_ptr(), 4, 8192, _hip._stream(x))
    assert st == 3  # RV_ERR_UNSUPPORTED: width above the 4096 the scratch is sized for
    # width <= 256: one partial row per 128 rows at this size; 524289 rows need
    # 4097 rows of 256 floats, one more than the 4 MiB scratch holds (rejected
    # before any launch)
    st = lib.rv_rmsnorm_bwd_noalloc(x.data_ptr(), w.data_ptr(), x.data_ptr(), rstd.data_ptr(),
                                    x.data_ptr(), w.data_ptr(), 524289, 256, _hip._stream(x))
    assert st == 4  # RV_ERR_WORKSPACE
    assert lib.rv_rmsnorm_bwd_noalloc(None, w.data_ptr(), x.data_ptr(), rstd.data_ptr(),
                                      x.data_ptr(), w.data_ptr(), 4, 256, None) == 1
    assert lib.rv_rmsnorm_bwd_noalloc(ctypes.c_void_p(x.data_ptr()), w.data_ptr(), x.data_ptr(),
                                      rstd.data_ptr(), x.data_ptr(), w.data_ptr(), 0, 256,
                                      None) == 2


@pytest.mark.gpu
def test_noalloc_on_a_stream_of_the_current_device(cuda_device):
    """A non-default stream of the current device is accepted (the entry point
    checks the stream's device against the current one) and gives the same bits."""
    lib = _hip.library()
    x, w, dy, rstd = _inputs(2048, 256, 7, cuda_device)
    ref_dx, ref_dw = _with_workspace(lib, x, w, dy, rstd)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=cuda_device)
    dx = torch.full_like(x, float("nan"))
    dw = torch.full_like(w, float("nan"))
    st = lib.rv_rmsnorm_bwd_noalloc(x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(),
                                    dx.data_ptr(), dw.data_ptr(), 2048, 256, side.cuda_stream)
    assert st == 0, lib.rv_status_string(st)
    side.synchronize()
    assert torch.equal(dx, ref_dx) and torch.equal(dw, ref_dw)


_CAPTURE_CHILD = textwrap.dedent("""
    import sys
    sys.path.insert(0, sys.argv[1])
    import torch
    from reversability_amd import _hip
    lib = _hip.library()
    dev = torch.device("cuda", 0)
    eps = float(torch.finfo(torch.float32).eps)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(5000, 256, generator=g).to(dev)
    w = (1 + 0.02 * torch.randn(256, generator=g)).to(dev)
    dy = torch.randn(5000, 256, generator=g).to(dev)
    _, rstd = _hip.ops.rmsnorm_fwd(x, w, eps)
    nbytes = lib.rv_rmsnorm_bwd_workspace_bytes(5000, 256)
    ws = torch.empty(nbytes // 4, device=dev)
    ref_dx, ref_dw = torch.empty_like(x), torch.empty_like(w)
    assert lib.rv_rmsnorm_bwd(x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(),
                              ref_dx.data_ptr(), ref_dw.data_ptr(), ws.data_ptr(), nbytes,
                              5000, 256, _hip._stream(x)) == 0
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.rv_rmsnorm_bwd_noalloc(
            x.data_ptr(), w.data_ptr(), dy.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
            dw.data_ptr(), 5000, 256, torch.cuda.current_stream().cuda_stream)
    assert status == 0, (status, lib.rv_last_error())
    for replay in range(3):
        dx.fill_(float("nan"))
        dw.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, ref_dx) and torch.equal(dw, ref_dw), replay
    print("replays equal", flush=True)
""")


@pytest.mark.gpu
def test_noalloc_first_call_under_graph_capture(cuda_device):
    """In a fresh process, the first call of rv_rmsnorm_bwd_noalloc -- the one
    that looks up the scratch array's device address -- is made inside a HIP
    graph capture; three replays (eager fills and synchronizations between
    them) give rv_rmsnorm_bwd's bits."""
    root = Path(__file__).resolve().parents[1]
    print("[noalloc] child process: first call under graph capture", flush=True)
    run = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, str(root)], capture_output=True,
                         text=True, timeout=240, cwd=str(root))
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-2000:]
    assert "replays equal" in run.stdout
