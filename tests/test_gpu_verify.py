"""The quantized layers of a batched verify forward, eager and captured in a HIP graph (needs an
MI355X).

Bars: the two-layer stack against the oracle's composition (fp32-accumulated projections, the
oracle's norm and SiLU·mul, bf16 between ops) to max_rel <= 1e-2 and mean_rel <= 2e-3 (ulp-level differences
of intermediate roundings propagate through the residual stream, so the whole chain is held to the
tolerance rather than to bits); graph replays bit-equal to eager calls on the same inputs.
"""

import numpy as np
import pytest
import torch

from mlx_tree_spec_amd import GraphedTail, MLPLayer, QuantizedLinear, QuantizedMLP, stack_tail
from oracle import cpu
from oracle import qmm4_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
D, H, EPS = 512, 1024, 1e-6


def bf16_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def u32_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(DEV)


def host_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def make_stack(n_layers=2, seed=0, d=D, hdim=H):
    rng = np.random.default_rng(seed)
    layers, ref = [], []

    def lin(n, k, s):
        _, w, sc, b = O.make_inputs(1, k, n, seed=s)
        return QuantizedLinear.from_quantized(u32_dev(w), bf16_dev(sc), bf16_dev(b)), (w, sc, b)

    def norm():
        wn = O.f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
        m = torch.nn.RMSNorm(d, eps=EPS, device=DEV, dtype=torch.bfloat16)
        with torch.no_grad():
            m.weight.copy_(bf16_dev(wn))
        return m, wn

    for i in range(n_layers):
        post, wpost = norm()
        g, gw = lin(hdim, d, 100 * seed + 10 * i + 1)
        u, uw = lin(hdim, d, 100 * seed + 10 * i + 2)
        dn, dw = lin(d, hdim, 100 * seed + 10 * i + 3)
        layers.append(MLPLayer(post, QuantizedMLP(g, u, dn)))
        gu = tuple(np.concatenate([a, c]) for a, c in zip(gw, uw))
        ref.append((wpost, gu, dw))
    final, wfinal = norm()
    return layers, final, ref, wfinal


def oracle_stack(h, rs, ref, wfinal):
    """The same layers on the CPU: oracle norm, fp32-accumulated projections rounded to bf16."""
    x = None
    for i, (wpost, gu, dw) in enumerate(ref):
        h, x = O.add_rms_norm(h, rs[i], wpost, EPS)
        t = O.f32_to_bf16_bits(cpu.qmm_f32(x, *gu))
        hh = t.shape[1] // 2
        a = O.silu_mul(t[:, :hh], t[:, hh:])
        mo = O.f32_to_bf16_bits(cpu.qmm_f32(a, *dw))
        wn = ref[i + 1][0] if i + 1 < len(ref) else wfinal
        h, x = O.add_rms_norm(h, mo, wn, EPS)
    return h, x


def inputs(rows, n_layers, seed, d=D):
    rng = np.random.default_rng(seed)
    h = O.f32_to_bf16_bits(rng.standard_normal((rows, d)).astype(np.float32))
    rs = [O.f32_to_bf16_bits((0.5 * rng.standard_normal((rows, d))).astype(np.float32)) for _ in range(n_layers)]
    return h, rs


# M = the sum of the requests' tree nodes: one decode request of 3 nodes (row-split kernels), and
# 4 requests x 16 nodes (verify kernels, two-pass gate+up); at a width of 1024 and 8192 MLP
# columns, 1 and 4 rows take the norm folded into the gate+up kernel.
@pytest.mark.parametrize("rows,d,hdim", [(3, D, H), (64, D, H), (1, 1024, 8192), (4, 1024, 8192)])
def test_stack_tail_matches_oracle_composition(rows, d, hdim):
    layers, final, ref, wfinal = make_stack(d=d, hdim=hdim)
    h, rs = inputs(rows, len(layers), rows, d)
    hg, xg = stack_tail(bf16_dev(h), [bf16_dev(r) for r in rs], layers, final)
    ho, xo = oracle_stack(h, rs, ref, wfinal)
    for got, want in ((hg, ho), (xg, xo)):
        g = O.bf16_bits_to_f32(host_bits(got)).astype(np.float64)
        w = O.bf16_bits_to_f32(want).astype(np.float64)
        print(f"  stack rows={rows}: max_rel={O.max_rel(g, w):.2e} mean_rel={O.mean_rel(g, w):.2e}", flush=True)
        assert O.max_rel(g, w) <= O.MAX_REL_TOL and O.mean_rel(g, w) <= O.MEAN_REL_TOL


def check_tail(got, want, what):
    for gt_, wt in zip(got, want):
        g = O.bf16_bits_to_f32(host_bits(gt_)).astype(np.float64)
        w = O.bf16_bits_to_f32(wt).astype(np.float64)
        print(f"  {what}: max_rel={O.max_rel(g, w):.2e} mean_rel={O.mean_rel(g, w):.2e}", flush=True)
        assert O.max_rel(g, w) <= O.MAX_REL_TOL and O.mean_rel(g, w) <= O.MEAN_REL_TOL


@pytest.mark.parametrize("rows,d,hdim", [(4, D, H), (64, D, H), (4, 1024, 8192)])
def test_graphed_tail_replays_equal_eager(rows, d, hdim):
    """Replays against the oracle's composition (not only against eager calls), with eager work of
    the same shape and of a larger shape on other streams between the replays."""
    layers, final, ref, wfinal = make_stack(seed=1, d=d, hdim=hdim)
    gt = GraphedTail(layers, final, rows, d, DEV)
    side = torch.cuda.Stream()
    for rep in range(3):
        h, rs = inputs(rows, len(layers), 1000 * rows + rep, d)
        hd, rsd = bf16_dev(h), [bf16_dev(r) for r in rs]
        he, xe = stack_tail(hd, rsd, layers, final)  # eager work between the replays
        he, xe = host_bits(he), host_bits(xe)
        # A larger batch on another stream: its split-K workspace and scratch are that stream's.
        hb, rsb = inputs(2 * rows + 7, len(layers), 7 + rep, d)
        with torch.cuda.stream(side):
            stack_tail(bf16_dev(hb), [bf16_dev(r) for r in rsb], layers, final)
        side.synchronize()
        torch.cuda.synchronize()
        hr, xr = gt(hd, rsd)
        torch.cuda.synchronize()
        assert np.array_equal(host_bits(hr), he), f"replay {rep}: h differs from eager"
        assert np.array_equal(host_bits(xr), xe), f"replay {rep}: x differs from eager"
        check_tail((hr, xr), oracle_stack(h, rs, ref, wfinal), f"replay {rep} rows={rows} vs oracle")
