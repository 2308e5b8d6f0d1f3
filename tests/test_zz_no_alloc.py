"""The no-allocation entry point qmm4_affine_bf16_noalloc through the C ABI (needs an MI355X).

Bar: bit-identical to qmm4_affine_bf16 (the same kernels; only where the split-K workspace lives
differs), on two calls in a row of each kernel family that uses the workspace, the second with a
smaller input; the results also meet the parity tolerance against the oracle. The defining
property, that no call allocates, is checked twice: free device memory (hipMemGetInfo) does not
move across eager calls that need a workspace on a brand-new stream, and such a call captured on a
brand-new stream succeeds where qmm4_affine_bf16 returns QMM4_ERR_CAPTURE (it would have to
allocate). The first test also records when the static array is reserved: at the first call on a
device, not when the library is loaded.
"""

import numpy as np
import pytest
import torch

from mlx_tree_spec_amd import _lib
from oracle import qmm4_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a).view(dt)).to(DEV)


def run(fn, x, w, s, b, m, n, k, stream):
    xd, wd, sd, bd = dev(x, np.int16), dev(w, np.int32), dev(s, np.int16), dev(b, np.int16)
    y = torch.full((m, n), -1, dtype=torch.int16, device=DEV)
    rc = fn(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y.data_ptr(), m, n, k, 64, 4, 1, stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16)


MIB = 1 << 20


def free_bytes():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]


def test_noalloc_first_call_reserves_the_array():
    """The library's static array (QMM4_NOALLOC_SCRATCH_BYTES per GPU) takes device memory at the
    first qmm4_affine_bf16_noalloc call on a device (its code object is loaded when the array's
    address is looked up), not when the library is loaded or its other entry points run. Measured
    in this process when no earlier test made a no-alloc call (this file is collected last)."""
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    m, n, k = 1, 512, 512  # row-split over whole K: no workspace
    x, w, s, b = O.make_inputs(m, k, n, seed=3)
    run(lib.qmm4_affine_bf16, x, w, s, b, m, n, k, stream)
    before = free_bytes()
    got = run(lib.qmm4_affine_bf16_noalloc, x, w, s, b, m, n, k, stream)
    after = free_bytes()
    again = run(lib.qmm4_affine_bf16_noalloc, x, w, s, b, m, n, k, stream)
    after2 = free_bytes()
    delta = before - after
    print(f"  free device memory: {before / MIB:.1f} MiB before the first no-alloc call, "
          f"{after / MIB:.1f} MiB after it (delta {delta / MIB:.1f} MiB), {after2 / MIB:.1f} MiB after the second",
          flush=True)
    assert np.array_equal(got, again)
    assert after2 == after, "a second no-alloc call changed free device memory"
    # Reserved here (the first call in this process), or already by an earlier no-alloc call.
    assert delta == 0 or _lib.QMM4_NOALLOC_SCRATCH_BYTES <= delta <= _lib.QMM4_NOALLOC_SCRATCH_BYTES + 64 * MIB


def test_noalloc_allocates_nothing_on_new_streams():
    """Eager calls of a shape that needs a split-K workspace (row-phase K split, 15.7 MB of partial
    tiles; stream-K GEMM) on a brand-new stream: no change in free device memory, where the
    allocating entry point grows a workspace for the new stream."""
    lib = _lib.load()
    shapes = [(64, 5120, 17408), (128, 17408, 5120)]
    data = []
    for m, n, k in shapes:
        x, w, s, b = O.make_inputs(m, k, n, seed=11 + m)
        xd, wd, sd, bd = dev(x, np.int16), dev(w, np.int32), dev(s, np.int16), dev(b, np.int16)
        y = torch.zeros((m, n), dtype=torch.int16, device=DEV)
        data.append((m, n, k, xd, wd, sd, bd, y))

    def call(fn, d, stream):
        m, n, k, xd, wd, sd, bd, y = d
        rc = fn(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y.data_ptr(), m, n, k, 64, 4, 1, stream)
        assert rc == 0, _lib.last_error()

    # Kernels loaded and the array set up on the default stream first.
    for d in data:
        call(lib.qmm4_affine_bf16_noalloc, d, torch.cuda.current_stream().cuda_stream)
    want = [d[-1].clone() for d in data]

    def new_stream():
        # HIP sets up a stream's hardware queue (a few MiB of device memory) at its first use, so
        # each new stream runs a small torch op before free memory is read.
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            torch.ones(1, device=DEV).add_(1)
        st.synchronize()
        return st

    st = new_stream()
    before = free_bytes()
    for d in data:
        call(lib.qmm4_affine_bf16_noalloc, d, st.cuda_stream)
    st.synchronize()
    after = free_bytes()
    print(f"  no-alloc on a new stream: free device memory {before / MIB:.1f} -> {after / MIB:.1f} MiB", flush=True)
    assert after == before
    for d, wnt in zip(data, want):
        assert torch.equal(d[-1], wnt)
    # The allocating entry point on another new stream grows that stream's workspace.
    st2 = new_stream()
    after = free_bytes()
    call(lib.qmm4_affine_bf16, data[0], st2.cuda_stream)
    st2.synchronize()
    grown = free_bytes()
    print(f"  qmm4_affine_bf16 on a new stream: free device memory {after / MIB:.1f} -> {grown / MIB:.1f} MiB",
          flush=True)
    assert after - grown >= 15 * MIB
    assert torch.equal(data[0][-1], want[0])


def test_noalloc_captures_where_the_allocating_entry_cannot():
    """Captured on a brand-new stream, a shape that needs a workspace: qmm4_affine_bf16 returns
    QMM4_ERR_CAPTURE (its workspace for that stream would have to be allocated), the no-alloc entry
    point records its kernels, and the replays reproduce the eager result."""
    lib = _lib.load()
    m, n, k = 64, 5120, 17408
    x, w, s, b = O.make_inputs(m, k, n, seed=21)
    want = run(lib.qmm4_affine_bf16_noalloc, x, w, s, b, m, n, k, torch.cuda.current_stream().cuda_stream)
    xd, wd, sd, bd = dev(x, np.int16), dev(w, np.int32), dev(s, np.int16), dev(b, np.int16)
    y = torch.zeros((m, n), dtype=torch.int16, device=DEV)
    args = (xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y.data_ptr(), m, n, k, 64, 4, 1)
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        rc_alloc = lib.qmm4_affine_bf16(*args, st.cuda_stream)
        rc_noalloc = lib.qmm4_affine_bf16_noalloc(*args, st.cuda_stream)
    assert rc_alloc == _lib.QMM4_ERR_CAPTURE, rc_alloc
    assert rc_noalloc == 0, _lib.last_error()
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint16), want), f"replay {rep}"


# (larger shape, smaller shape) per kernel family that takes a split-K workspace: row-split with K
# slices (counters + partials), row-phase with a K split (partials), K-split verify (counters +
# partials), stream-K skinny (counters + partials); the GEMM's stream-K over 128 x 128 tiles on a
# few and on 256 workgroups (32 MiB of partials); its stream-K over 256 x 256 tiles (128 MiB of
# partials, the largest workspace), over the quarters of a last round of whole tiles, and over
# 128 x 256 tiles (64 MiB of partials).
PAIRS = [
    ((2, 5120, 17408), (1, 2048, 8192)),
    ((64, 5120, 17408), (24, 2048, 5120)),
    ((16, 512, 5120), (8, 256, 2048)),
    ((3, 256, 4096), (2, 64, 1024)),
    ((96, 640, 1024), (80, 256, 512)),
    ((512, 5120, 17408), (128, 17408, 5120)),
    ((1024, 17408, 5120), (96, 512, 1024)),
    ((256, 17408, 5120), (136, 10256, 5120)),  # stream-K over 128 x 256 tiles, then a partial one
]


@pytest.mark.parametrize("big,small", PAIRS)
def test_noalloc_matches_allocating_entry(big, small):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for i, (m, n, k) in enumerate((big, small)):
        print(f"  noalloc call {i}: M={m} N={n} K={k}", flush=True)
        x, w, s, b = O.make_inputs(m, k, n, seed=100 + i + m)
        got = run(lib.qmm4_affine_bf16_noalloc, x, w, s, b, m, n, k, stream)
        want = run(lib.qmm4_affine_bf16, x, w, s, b, m, n, k, stream)
        assert np.array_equal(got, want), f"call {i} M={m} N={n} K={k}: noalloc differs from qmm4_affine_bf16"
        ref = O.quantized_matmul_exact(x, w, s, b) if m * n * k <= 2 ** 28 else None
        if ref is not None:
            yf = O.bf16_bits_to_f32(got).astype(np.float64)
            assert O.max_rel(yf, ref) <= O.MAX_REL_TOL and O.mean_rel(yf, ref) <= O.MEAN_REL_TOL


def test_noalloc_on_side_stream_and_graph_replay():
    """After its first call a device's static scratch serves calls on any stream and under capture."""
    lib = _lib.load()
    m, n, k = 16, 512, 5120
    x, w, s, b = O.make_inputs(m, k, n, seed=7)
    want = run(lib.qmm4_affine_bf16, x, w, s, b, m, n, k, torch.cuda.current_stream().cuda_stream)
    xd, wd, sd, bd = dev(x, np.int16), dev(w, np.int32), dev(s, np.int16), dev(b, np.int16)
    y = torch.zeros((m, n), dtype=torch.int16, device=DEV)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        assert lib.qmm4_affine_bf16_noalloc(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                                            y.data_ptr(), m, n, k, 64, 4, 1, st.cuda_stream) == 0
    st.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        assert lib.qmm4_affine_bf16_noalloc(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                                            y.data_ptr(), m, n, k, 64, 4, 1, st.cuda_stream) == 0
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint16), want), f"replay {rep}"
