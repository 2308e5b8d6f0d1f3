"""Kernel planners against what their kernels assume (CPU only, no GPU call).

tests/plan_invariants.cpp calls the planners exported by the built libqmm4.so (row-split, its
x-in-registers form, row-phase, K-split verify, GEMM) over a grid of shapes (1-4096 rows, 16-262144 columns,
K = 128-20480) and CU counts (1-304), and checks every accepted plan: dynamic LDS within 160 KB,
output columns covered exactly once, K slices and units that tile K, each loop form only in the
configuration its launch path instantiates, stream-K workgroups between 1 and the unit count
within the workspace. The planners pick the kernel for the reference's quantized_matmul
(packed_linear.py:83-104 routes by rows), so a plan that broke one of these would launch a kernel
outside its assumptions.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "mlx-tree-spec_amd", "mlx_tree_spec_amd")
LIB = os.path.join(LIBDIR, "libqmm4.so")


@pytest.fixture(scope="module")
def planner_exe(tmp_path_factory):
    if not os.path.exists(LIB):
        pytest.skip("libqmm4.so is not built (run __graft_entry__.build())")
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ is not available")
    exe = tmp_path_factory.mktemp("plans") / "plan_invariants"
    cmd = [cxx, "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "mlx-tree-spec_amd", "csrc"),
           os.path.join(ROOT, "tests", "plan_invariants.cpp"), "-L", LIBDIR, "-lqmm4",
           f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stderr[-4000:]
    return str(exe)


def query(exe, lines):
    """The planners' forms for `lines` ("<planner> M N K cus" each), one output line per query."""
    run = subprocess.run([exe, "query"], input="".join(ln + "\n" for ln in lines), capture_output=True,
                         text=True, timeout=60)
    assert run.returncode == 0, run.stderr
    out = run.stdout.splitlines()
    assert len(out) == len(lines)
    return [dict(kv.split("=") for kv in o.split()) if "=" in o and not o.startswith("xreg") else o for o in out]


def test_planners_keep_kernel_invariants(planner_exe):
    exe = planner_exe
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-2000:]
    assert "violations: 0" in run.stdout
    checked = int(run.stdout.split("plans checked:")[1].split(",")[0])
    assert checked > 10000, run.stdout


def test_fold_cases_take_their_routes(planner_exe):
    """Each shape of test_gpu_norm_fold.py reaches the form its label names on 256 CUs: the folded
    row-split launch (4-row fragments, the regular form) with K whole or in 2 slices, or two
    launches. The fold runs when dispatch_norm_qmm's condition holds: at most 4 rows and a row-split
    plan (fused for the gate+up) that rowsplit_norm_ok accepts."""
    from route_cases import CUS, FOLD_CASES

    lines = [f"{'rowsplit_fused' if su else 'rowsplit'} {m} {n} {k} {CUS}" for m, n, k, su, _ in FOLD_CASES]
    for (m, n, k, su, route), p in zip(FOLD_CASES, query(planner_exe, lines)):
        folded = m <= 4 and isinstance(p, dict) and p["norm_ok"] == "1"
        if route == "two launches":
            assert not folded, (m, n, k, su, p)
        else:
            assert folded, (m, n, k, su, p)
            assert p["MP"] == "4" and p["small"] == "0" and p["pair"] == "0" and p["own"] == "0"
            assert route == f"fold KS={p['KS']}", (m, n, k, su, route, p)


def test_gate_up_cases_take_their_routes(planner_exe):
    """Each shape of test_gpu_mlp.py reaches its route on 256 CUs (dispatch_gate_up_silu): the fused
    row-split launch when rowsplit_plan(fused) accepts it; else, at 5-96 rows with K % 512 == 0 and
    no unfused row-split plan up to 16 rows, the fused row-phase launch (gate_up_routes); else the
    two-pass path."""
    from route_cases import GATE_UP_CASES

    routes = gate_up_routes(planner_exe, [(m, k, n) for m, k, n, _ in GATE_UP_CASES])
    for (m, k, n, route), want in zip(GATE_UP_CASES, routes):
        assert route == want, (m, k, n, route, want)


def test_random_gate_up_shapes_reach_every_route(planner_exe):
    """test_gpu_mlp.py's seeded random gate+up shapes reach each of the three routes several times."""
    from route_cases import RANDOM_GATE_UP

    routes = gate_up_routes(planner_exe, RANDOM_GATE_UP)
    for r in ("fused", "row-phase fused", "two-pass"):
        assert routes.count(r) >= 5, (r, routes)


def gate_up_routes(planner_exe, shapes):
    """dispatch_gate_up_silu's route for each (M, K, N) on 256 CUs, from the planners' answers: the
    fused row-split launch; else the row-phase plan the projection would take (5-96 rows, K % 512 ==
    0, no row-split or x-in-registers plan up to 16 rows), fused: a wide plan under the range-size
    rule, a narrow (K-split) plan where the projection takes it (17 rows or more, or a K split
    filling half the CUs); else the two passes."""
    from route_cases import CUS

    MAX_MK = 1 << 19
    nc = len(shapes)
    lines = [f"rowsplit_fused {m} {n} {k} {CUS}" for m, k, n in shapes]
    lines += [f"rowphase_fused {m} {n} {k} {CUS}" for m, k, n in shapes]
    lines += [f"rowsplit {m} {n} {k} {CUS}" for m, k, n in shapes]
    lines += [f"rowphase {m} {n} {k} {CUS}" for m, k, n in shapes]
    lines += [f"xreg {m} {n} {k} {CUS}" for m, k, n in shapes]
    out = query(planner_exe, lines)
    routes = []
    for i, (m, k, n) in enumerate(shapes):
        rs, rp, rsp, ru, xr = out[i], out[nc + i], out[2 * nc + i], out[3 * nc + i], out[4 * nc + i]
        take = False
        if (rs == "none" and 5 <= m <= 96 and k % 512 == 0 and isinstance(rp, dict) and isinstance(ru, dict)
                and not (m <= 16 and (rsp != "none" or (m >= 9 and xr != "none")))):
            if rp["wide"] == "1":
                assert rp["S"] == "1", (m, k, n, rp)
                take = ((m <= 64 or int(rp["blocks"]) <= CUS)
                        and (int(rp["BW"]) <= int(ru["BW"]) or (m >= 17 and m * k <= MAX_MK)))
            else:  # the projection's own K-split plan
                assert {key: rp[key] for key in ("variant", "S", "BW", "blocks")} == \
                    {key: ru[key] for key in ("variant", "S", "BW", "blocks")}, (m, k, n, rp, ru)
                take = m >= 17 or 2 * int(rp["blocks"]) >= CUS
        routes.append("fused" if rs != "none" else "row-phase fused" if take else "two-pass")
    return routes


def test_mid_row_cases_take_their_routes(planner_exe):
    """Each 65-128-row shape of test_gpu_parity.py reaches its route on 256 CUs: the row-phase
    kernel when dispatch_qmm's condition holds (up to 112 rows, or 128 over at most 2048 columns;
    K % 512 == 0; a narrow row-phase plan, or up to 96 rows a wide one of at most one range per
    CU), else the GEMM."""
    from route_cases import CUS, MID_ROW_CASES

    lines = [f"rowphase {m} {n} {k} {CUS}" for m, n, k, _ in MID_ROW_CASES]
    for (m, n, k, route), p in zip(MID_ROW_CASES, query(planner_exe, lines)):
        rows_ok = m <= 112 or (m <= 128 and n <= 2048)
        plan_ok = isinstance(p, dict) and (p["wide"] == "0" or (m <= 96 and int(p["blocks"]) <= CUS))
        takes = rows_ok and k % 512 == 0 and plan_ok
        assert route == ("row-phase" if takes else "gemm"), (m, n, k, route, p)


def test_rowphase_wide_cases_take_their_variants(planner_exe):
    """Each wide row-phase shape of test_gpu_parity.py reaches the variant form its label names on
    256 CUs: a variant whose short waves skip the last block slot ("opt", ids 20-23 of the kernel
    table) or one that computes every slot ("full")."""
    from route_cases import CUS, ROWPHASE_WIDE_CASES

    lines = [f"rowphase {m} {n} {k} {CUS}" for m, n, k, _ in ROWPHASE_WIDE_CASES]
    for (m, n, k, form), p in zip(ROWPHASE_WIDE_CASES, query(planner_exe, lines)):
        assert isinstance(p, dict) and p["wide"] == "1" and p["S"] == "1", (m, n, k, p)
        assert (20 <= int(p["variant"]) <= 23) == (form == "opt"), (m, n, k, form, p)


def test_random_shapes_keep_kernel_invariants(planner_exe):
    """The seeded random shapes of test_gpu_parity.py (RANDOM_SHAPES) pass every planner's checks
    at 256, 304 and 80 CUs before any of them runs on a GPU."""
    import ast

    src = open(os.path.join(ROOT, "tests", "test_gpu_parity.py")).read()
    start = src.index("RANDOM_SHAPES = ")
    shapes = ast.literal_eval(src[start + len("RANDOM_SHAPES = "):src.index("]", start) + 1])
    assert len(shapes) >= 40
    run = subprocess.run([planner_exe, "check"], input="".join(f"{m} {n} {k}\n" for m, k, n in shapes),
                         capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-2000:]
    assert "violations: 0" in run.stdout


def dispatch_route(exe, cases):
    """dispatch_qmm's route for each (M, N, K) on 256 CUs with 16-byte aligned scales, from the
    built planners queried in dispatch order: past 64 rows the row-phase kernel (narrow plans up to
    112 rows or 128 over at most 2048 columns, wide plans of at most one range per CU up to 96
    rows) else the GEMM; up to 64 rows the x-in-registers row-split form (9-16 rows), the row-split
    kernel, the row-phase kernel (from 5 rows when its plan is wide, has 17+ rows or fills half the
    CUs), else the verify or skinny kernel ("other")."""
    from route_cases import CUS

    kinds = ("rowphase", "xreg", "rowsplit")
    lines = [f"{kind} {m} {n} {k} {CUS}" for m, n, k in cases for kind in kinds]
    out = query(exe, lines)
    routes = []
    for i, (m, n, k) in enumerate(cases):
        rp, xr, rs = out[3 * i:3 * i + 3]
        rp_ok = isinstance(rp, dict) and k % 512 == 0
        if m > 64:
            rows_ok = m <= 112 or (m <= 128 and n <= 2048)
            wide_ok = rp_ok and (rp["wide"] == "0" or (m <= 96 and int(rp["blocks"]) <= CUS))
            routes.append("row-phase" if rows_ok and wide_ok else "gemm")
        elif m >= 9 and xr != "none":
            routes.append("xreg")
        elif rs != "none":
            routes.append("row-split")
        elif m >= 5 and rp_ok and (rp["wide"] == "1" or m >= 17 or 2 * int(rp["blocks"]) >= CUS):
            routes.append("row-phase")
        else:
            routes.append("other")
    return routes


def test_rowphase_test_shapes_reach_the_rowphase_kernel(planner_exe):
    """Every shape of the row-phase tests in test_gpu_parity.py (shapes, one-hot exact dequant,
    window form switches, the wide variants) is sent to the row-phase kernel by dispatch_qmm."""
    from route_cases import ROWPHASE_ONE_HOT, ROWPHASE_SHAPES, ROWPHASE_WIDE_CASES, ROWPHASE_WINDOW_CASES

    cases = ([(m, n, k) for m, k, n in ROWPHASE_SHAPES] + [(m, n, k) for n, m, k in ROWPHASE_ONE_HOT]
             + [(m, n, k) for m, k, n in ROWPHASE_WINDOW_CASES] + [(m, n, k) for m, n, k, _ in ROWPHASE_WIDE_CASES])
    for case, route in zip(cases, dispatch_route(planner_exe, cases)):
        assert route == "row-phase", (case, route)


def test_gemm_stream_k_cases_take_their_tiles(planner_exe):
    """Each GEMM stream-K shape of test_gpu_parity.py runs on the tile size its label names."""
    from route_cases import CUS, GEMM_STREAM_K_CASES

    lines = [f"gemm {m} {n} {k} {CUS}" for m, n, k, _ in GEMM_STREAM_K_CASES]
    for (m, n, k, tiles), p in zip(GEMM_STREAM_K_CASES, query(planner_exe, lines)):
        assert p["sk"] == "1" and p["sk256"] == "0", (m, n, k, p)
        assert p["sk_wide"] == ("1" if tiles == "128x256" else "0"), (m, n, k, tiles, p)
