"""fgmm_iso_estep_f32_noalloc (workspace in the library's fixed device scratch) against
fgmm_iso_estep_f32 (workspace allocated by the caller), both through the C ABI."""

import os
import sys

import pytest
import torch

from flash_gmm import _lib, data
from oracle import gmm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from parity import assert_close_stats  # noqa: E402

pytestmark = pytest.mark.gpu


def _inputs(inp, dev):
    return [inp[k].to(dev).contiguous() for k in ("X", "mu", "log_sigma_sq", "log_pi")]


def _outputs(N, K, D, dev):
    nan = float("nan")
    return [torch.full((N,), nan, device=dev), torch.full((K,), nan, device=dev),
            torch.full((K, D), nan, device=dev), torch.full((K,), nan, device=dev)]


def _run(inp, dev, noalloc, flags=0, outs=None):
    L = _lib.lib()
    X, mu, lss, lpi = _inputs(inp, dev)
    N, D = X.shape
    K = mu.shape[0]
    o = outs if outs is not None else _outputs(N, K, D, dev)
    ptrs = [t.data_ptr() for t in o]
    if flags & _lib.FLAG_NO_LOGZ:
        ptrs[0] = None
    stream = _lib.stream_handle(dev)
    if noalloc:
        st = L.fgmm_iso_estep_f32_noalloc(X.data_ptr(), D, N, D, mu.data_ptr(), D, K, lss.data_ptr(),
                                          lpi.data_ptr(), *ptrs, flags, stream)
    else:
        ws = torch.empty(max(1, L.fgmm_iso_workspace_bytes_ex(N, K, D, flags)), dtype=torch.uint8, device=dev)
        st = L.fgmm_iso_estep_f32(X.data_ptr(), D, N, D, mu.data_ptr(), D, K, lss.data_ptr(),
                                  lpi.data_ptr(), *ptrs, ws.data_ptr(), ws.numel(), flags, stream)
    _lib.check(st, "noalloc" if noalloc else "workspace")
    torch.cuda.synchronize()
    return o


def test_scratch_is_reserved_by_the_first_noalloc_call(gpu_device):
    """The scratch array is its own code object's: HIP loads that code object on its first
    use, the first noalloc call's symbol lookup, so a process that only calls the
    workspace entry points does not reserve it.  Measured as the device's free memory
    around the first noalloc call of this process (none ran before this test's call:
    this file runs last and this test only the workspace entry point before it)."""
    dev = gpu_device
    inp = data.iso_clustered(3000, 64, 32, seed=35)
    _run(inp, dev, noalloc=False)                   # the isotropic kernels are loaded
    X, mu, lss, lpi = _inputs(inp, dev)
    o = _outputs(3000, 64, 32, dev)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info(dev)
    L = _lib.lib()
    st = L.fgmm_iso_estep_f32_noalloc(X.data_ptr(), 32, 3000, 32, mu.data_ptr(), 32, 64, lss.data_ptr(),
                                      lpi.data_ptr(), *[t.data_ptr() for t in o], 0, _lib.stream_handle(dev))
    _lib.check(st, "noalloc")
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info(dev)
    print(f"device free memory around the first noalloc call: {free0} -> {free1} "
          f"({(free0 - free1) / 2**20:.1f} MiB)", flush=True)
    if os.environ.get("HIP_ENABLE_DEFERRED_LOADING", "1") != "0":
        assert free0 - free1 >= 64 << 20


def test_noalloc_equals_the_workspace_entry_point_on_two_calls(gpu_device):
    """Two calls in a row on one GPU's scratch, the second smaller (fewer rows, blocks
    and dimensions): each bitwise equal to the workspace entry point, the second also
    against the float64 oracle."""
    first = data.iso_clustered(60000, 512, 128, seed=31)
    second = data.iso_clustered(5000, 300, 64, seed=32)
    for inp in (first, second):
        ref = _run(inp, gpu_device, noalloc=False)
        got = _run(inp, gpu_device, noalloc=True)
        for u, v in zip(got, ref):
            assert torch.equal(u, v)
    assert_close_stats(got, O.estep_iso(*[second[k] for k in ("X", "mu", "log_sigma_sq", "log_pi")]),
                       "noalloc")


def test_noalloc_phase_split_and_bf16(gpu_device):
    inp = data.iso_clustered(8000, 256, 96, seed=33)
    dev = gpu_device
    ref = _run(inp, dev, noalloc=False)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = _outputs(N, K, D, dev)
    _run(inp, dev, noalloc=True, flags=_lib.FLAG_PHASE1, outs=out)
    _run(inp, dev, noalloc=True, flags=_lib.FLAG_PHASE2 | _lib.FLAG_NO_LOGZ, outs=out)
    for u, v in zip(out, ref):
        assert torch.equal(u, v)
    b_ref = _run(inp, dev, noalloc=False, flags=_lib.FLAG_BF16)
    b_got = _run(inp, dev, noalloc=True, flags=_lib.FLAG_BF16)
    for u, v in zip(b_got, b_ref):
        assert torch.equal(u, v)


def test_noalloc_runs_row_chunks_beyond_its_scratch(gpu_device):
    """Beyond FGMM_NOALLOC_SCRATCH_BYTES of one call's workspace the entry point runs
    consecutive row chunks on its array: logZ bitwise the workspace entry point's (a
    row's log-normaliser does not depend on the other rows), the statistics to float32
    rounding (they are added once per chunk), and against invariants of all rows."""
    L = _lib.lib()
    dev = gpu_device
    N, K, D = 3_000_000, 1024, 128
    assert L.fgmm_iso_workspace_bytes(N, K, D) > 64 << 20
    inp = data.iso_clustered(N, K, D, seed=36, device=dev)
    ref = _run(inp, dev, noalloc=False)
    got = _run(inp, dev, noalloc=True)
    assert torch.equal(got[0], ref[0])
    for u, v in zip(got[1:], ref[1:]):
        assert float((u - v).abs().max()) <= 1e-5 * float(v.abs().max())
    assert abs(got[1].double().sum().item() - N) <= 1e-5 * N
    torch.testing.assert_close(got[2].double().sum(0), inp["X"].double().sum(0), rtol=1e-5,
                               atol=1e-5 * float(got[2].abs().sum(0).max()))


def test_noalloc_rejects_what_does_not_fit(gpu_device):
    """A phase-split call beyond FGMM_NOALLOC_SCRATCH_BYTES of workspace (it cannot span
    row chunks): FGMM_ERR_SCRATCH, nothing launched; the stored log-joint:
    FGMM_ERR_INVALID_ARG."""
    L = _lib.lib()
    dev = gpu_device
    N, K, D = 4_000_000, 1024, 128
    assert L.fgmm_iso_workspace_bytes(N, K, D) > 64 << 20
    X = torch.zeros(N, D, device=dev)
    mu = torch.zeros(K, D, device=dev)
    lss, lpi = torch.zeros(K, device=dev), torch.zeros(K, device=dev)
    o = _outputs(N, K, D, dev)
    for ph in (_lib.FLAG_PHASE1, _lib.FLAG_PHASE2):
        st = L.fgmm_iso_estep_f32_noalloc(X.data_ptr(), D, N, D, mu.data_ptr(), D, K, lss.data_ptr(),
                                          lpi.data_ptr(), *[t.data_ptr() for t in o], ph,
                                          _lib.stream_handle(dev))
        assert st == _lib.FGMM_ERR_SCRATCH
    assert "scratch" in L.fgmm_strerror(st).decode()
    torch.cuda.synchronize()
    assert torch.isnan(o[1]).all()   # nothing was written
    small = data.iso_clustered(100, 40, 32, seed=34)
    Xs, mus, lsss, lpis = _inputs(small, dev)
    os_ = _outputs(100, 40, 32, dev)
    st = L.fgmm_iso_estep_f32_noalloc(Xs.data_ptr(), 32, 100, 32, mus.data_ptr(), 32, 40, lsss.data_ptr(),
                                      lpis.data_ptr(), *[t.data_ptr() for t in os_],
                                      _lib.FLAG_STORE_LOGJOINT, _lib.stream_handle(dev))
    assert st == _lib.FGMM_ERR_INVALID_ARG
    torch.cuda.synchronize()
    assert torch.isnan(os_[1]).all()   # nothing was written


def test_noalloc_under_graph_capture(gpu_device):
    """The entry point captured into a HIP graph (torch.cuda.graph) after one warm-up
    call: each replay, with new inputs copied into the captured buffers and eager work
    and synchronisations between replays, bitwise equal to fgmm_iso_estep_f32 on the
    same inputs."""
    dev = gpu_device
    N, K, D = 20000, 256, 128
    sets = [data.iso_clustered(N, K, D, seed=40 + i) for i in range(3)]
    X, mu, lss, lpi = _inputs(sets[0], dev)
    o = _outputs(N, K, D, dev)
    L = _lib.lib()

    def call():
        st = L.fgmm_iso_estep_f32_noalloc(X.data_ptr(), D, N, D, mu.data_ptr(), D, K, lss.data_ptr(),
                                          lpi.data_ptr(), *[t.data_ptr() for t in o], 0,
                                          _lib.stream_handle(dev))
        _lib.check(st, "noalloc")

    call()                                 # warm-up: symbol lookup and kernel attributes
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    torch.cuda.synchronize()
    for rep in range(4):
        inp = sets[rep % 3]
        src = _inputs(inp, dev)
        for dst, s in zip((X, mu, lss, lpi), src):
            dst.copy_(s)
        for t in o:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = _run(inp, dev, noalloc=False)
        for u, v in zip(o, ref):
            assert torch.equal(u, v), f"replay {rep}"
