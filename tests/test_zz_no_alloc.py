"""The no-allocation entry point qmm4_affine_bf16_noalloc through the C ABI (needs an MI355X).

Bar: bit-identical to qmm4_affine_bf16 (the same kernels; only where the split-K workspace lives
differs), on two calls in a row of each kernel family that uses the workspace, the second with a
smaller input; the results also meet the parity tolerance against the oracle.
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


# (larger shape, smaller shape) per kernel family that takes a split-K workspace: row-split with K
# slices (counters + partials), row-phase with a K split (partials), K-split verify (counters +
# partials), stream-K skinny (counters + partials); the GEMM's stream-K over 128 x 128 tiles on a
# few and on 256 workgroups (32 MiB of partials); its stream-K over 256 x 256 tiles (128 MiB of
# partials, the largest workspace) and over the quarters of a last round of whole tiles.
PAIRS = [
    ((2, 5120, 17408), (1, 2048, 8192)),
    ((64, 5120, 17408), (24, 2048, 5120)),
    ((16, 512, 5120), (8, 256, 2048)),
    ((3, 256, 4096), (2, 64, 1024)),
    ((96, 512, 1024), (80, 256, 512)),
    ((512, 5120, 17408), (128, 17408, 5120)),
    ((1024, 17408, 5120), (96, 512, 1024)),
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
