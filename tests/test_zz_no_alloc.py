"""The allocation-free W8A8 linear (nq_linear_w8a8_noalloc) against the
workspace entry it mirrors (nq_linear_w8a8), called through the C ABI: the same
kernels, so the outputs are bit-identical. Two calls in a row on each case, the
second with a smaller input (the static scratch keeps the first call's contents,
which must not leak into the second); a shape beyond the scratch is refused
before anything is enqueued."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else t.data_ptr()


def _run_both(lib, dev, m, n, k, seed, bias, y_dt):
    from nanoinfer_amd import _lib
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn((m, k), generator=g, device=dev).half()
    wq = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
    ws = torch.rand(n, generator=g, device=dev) * 1e-3
    b = torch.randn(n, generator=g, device=dev) if bias else None
    ydt = torch.float16 if y_dt == _lib.NQ_F16 else torch.float32
    s = torch.cuda.current_stream().cuda_stream
    need = lib.nq_linear_w8a8_workspace_size(m, n, k)
    work = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    y_ref = torch.full((m, n), float("nan"), dtype=ydt, device=dev)
    st = lib.nq_linear_w8a8(_ptr(x), _lib.NQ_F16, _ptr(wq), _ptr(ws), _ptr(b), _ptr(y_ref), y_dt, m, n, k,
                            _ptr(work), work.numel(), 0, s)
    assert st == _lib.NQ_OK, lib.nq_last_error()
    y = torch.full((m, n), float("nan"), dtype=ydt, device=dev)
    st = lib.nq_linear_w8a8_noalloc(_ptr(x), _lib.NQ_F16, _ptr(wq), _ptr(ws), _ptr(b), _ptr(y), y_dt, m, n, k, 0, s)
    assert st == _lib.NQ_OK, lib.nq_last_error()
    torch.cuda.synchronize()
    return y, y_ref


# (large call, smaller follow-up): GEMV (m <= 2), skinny MFMA (m <= 64, with and
# without split K), wide tiles, prefill with split-K partial planes in the scratch
@pytest.mark.parametrize("big,small", [((2, 4864, 896), (1, 1536, 512)),
                                       ((64, 8960, 1536), (16, 1536, 1536)),
                                       ((32, 1536, 8960), (8, 256, 1536)),
                                       ((512, 1536, 8960), (300, 1000, 960)),
                                       ((2048, 8960, 1536), (200, 1003, 192))])
@pytest.mark.parametrize("y_dt", [0, 1])
def test_noalloc_matches_workspace_entry(dev, big, small, y_dt):
    from nanoinfer_amd import _lib
    lib = _lib.load()
    for i, (m, n, k) in enumerate((big, small)):
        y, y_ref = _run_both(lib, dev, m, n, k, seed=m + n + k + i, bias=i == 0, y_dt=y_dt)
        assert torch.isfinite(y_ref).all()
        assert torch.equal(y.view(torch.int16 if y.dtype == torch.float16 else torch.int32),
                           y_ref.view(torch.int16 if y.dtype == torch.float16 else torch.int32)), (m, n, k)


def test_noalloc_refuses_beyond_scratch(dev):
    from nanoinfer_amd import _lib
    lib = _lib.load()
    cap = lib.nq_linear_w8a8_noalloc_max_scratch()
    assert cap == 32 << 20
    m, n, k = 4096, 64, 8960                   # m * k alone is 35 MiB
    assert lib.nq_linear_w8a8_workspace_size(m, n, k) > cap
    x = torch.zeros((m, k), dtype=torch.float16, device=dev)
    wq = torch.zeros((n, k), dtype=torch.int8, device=dev)
    ws = torch.ones(n, device=dev)
    y = torch.full((m, n), 7.0, dtype=torch.float16, device=dev)
    st = lib.nq_linear_w8a8_noalloc(_ptr(x), _lib.NQ_F16, _ptr(wq), _ptr(ws), None, _ptr(y), _lib.NQ_F16, m, n, k,
                                    0, torch.cuda.current_stream().cuda_stream)
    assert st == _lib.NQ_BAD_SHAPE
    assert b"static buffer holds" in lib.nq_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())              # nothing was enqueued
    np.testing.assert_equal(lib.nq_linear_w8a8_noalloc(None, 0, None, None, None, None, 0, 0, n, k, 0, None), 0)


def test_noalloc_allocates_nothing_and_replays_in_a_graph(dev):
    """The property the entry exists for: a warm call changes no device
    allocation (free bytes before == after), and the call records into a HIP
    graph (capture refuses hipMalloc) whose replays, with eager work on y in
    between, each equal the eager call."""
    from nanoinfer_amd import _lib
    lib = _lib.load()
    m, n, k = 64, 8960, 1536
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn((m, k), generator=g, device=dev).half()
    wq = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
    ws = torch.rand(n, generator=g, device=dev) * 1e-3
    y = torch.empty((m, n), dtype=torch.float16, device=dev)
    s = torch.cuda.Stream()

    def call():
        st = lib.nq_linear_w8a8_noalloc(_ptr(x), _lib.NQ_F16, _ptr(wq), _ptr(ws), None, _ptr(y), _lib.NQ_F16,
                                        m, n, k, 0, torch.cuda.current_stream().cuda_stream)
        assert st == _lib.NQ_OK, lib.nq_last_error()
    with torch.cuda.stream(s):
        call()                                          # first call on the device: set-up
    torch.cuda.synchronize()
    ref = y.clone()
    free0 = torch.cuda.mem_get_info()[0]
    with torch.cuda.stream(s):
        call()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        call()
    for i in range(3):
        y.fill_(float(i + 1))                           # eager work between replays
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), i
