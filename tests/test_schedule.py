"""The program order of a launch, checked on the CPU: every program runs exactly once.

The kernel picks its program with program_of and the dynamic tail's ticket rules
(csrc/attn_fwd_schedule.hpp), which are __host__ __device__; the measurement library runs that
same code on the CPU for a whole launch (fa2_ablate_program_map), the tail's tickets taken in a
seeded random order with the kernel's wrapping increments emulated. This file sweeps thousands of
launch shapes (units, q tiles, GQA group, packing, unit chunk, causal or not, tail or static
order) on several device topologies and requires:

  * the library's map equals the numpy restatement (oracle/schedule.py) workgroup for workgroup on
    the static part, and as a set on the tail, with the same tail policy numbers;
  * every program of the grid runs exactly once (coverage_errors), spare tail workgroups run
    nothing, and every ticket word is back at zero after the launch;
  * planted mistakes in the restatement (an off-by-one in the unit chunk, in the reversed second
    round, in the tail's private blocks) fail the same coverage check on the same sweep.

The reference's CI likewise runs its kernel's index math on the CPU (tests/test_correctness.py:
83-87, under TRITON_INTERPRET). No GPU call anywhere here.
"""

import ctypes
import os

import numpy as np
import pytest

from oracle import schedule as sch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ABLATE_LIB = os.path.join(ROOT, "triton-fa2-forward_amd", "libfa2_ablate.so")
needs_ablate = pytest.mark.skipif(not os.path.exists(ABLATE_LIB), reason="libfa2_ablate.so not built")

INFO_WORDS = 11
# (CUs, XCDs): MI355X; MI300X (38 CUs per XCD); a CPX partition (one XCD); four and two XCDs;
# counts the order takes as one XCD (not a power of two; more than 16)
TOPOLOGIES = [(256, 8), (304, 8), (32, 1), (128, 4), (64, 2), (228, 6), (256, 32)]


def _map_fn():
    from ablation import ablate_lib

    fn = ablate_lib().fa2_ablate_program_map
    i32 = ctypes.c_int32
    fn.restype = ctypes.c_int
    fn.argtypes = [i32] * 12 + [ctypes.c_uint32, ctypes.POINTER(i32), ctypes.c_int64,
                                ctypes.POINTER(i32), i32]
    return fn


def library_map(fn, shape, seed=0, private_pct=-1):
    B, hq, hkv, n, d, causal, pack, bm, cus, xcds, static = shape
    groups = B * (hq // pack) * ((n * pack + bm - 1) // bm)
    cap = 3 * (groups + groups // 10 + 64)
    out = np.full(cap, -7, dtype=np.int32)
    info = np.zeros(INFO_WORDS, dtype=np.int32)
    rc = fn(B, hq, hkv, n, d, causal, pack, bm, cus, xcds, static, private_pct, seed,
            out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), cap,
            info.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), INFO_WORDS)
    assert rc == 0, shape
    grid = int(info[0])
    return out[: 3 * grid].reshape(grid, 3), dict(
        grid=grid, static_blocks=int(info[1]), tail_wgs=int(info[2]), queues=int(info[3]),
        private=int(info[4]), shared=int(info[5]), unit_chunk=int(info[6]),
        xcd_shift=int(info[7]), nonzero_words=int(info[8]), n_tiles=int(info[9]),
        n_bh=int(info[10]))


def sweep_shapes(count=3000, seed=1):
    """Launch shapes: the BASELINE configs and the tail tests' shapes on every topology, then
    seeded random ones (grids of at most ~40000 programs)."""
    fixed = [(1, 32, 8, 8192, 128, 1, 1, 128), (4, 16, 16, 4096, 128, 1, 1, 128),
             (2, 16, 16, 16384, 64, 0, 1, 128), (3, 28, 4, 1000, 128, 1, 1, 128),
             (3, 28, 4, 1000, 128, 1, 7, 112), (8, 16, 16, 4096, 128, 1, 1, 128),
             (4, 16, 16, 4096, 64, 1, 1, 128), (2, 32, 8, 2048, 128, 1, 4, 128),
             (3, 28, 4, 4096, 128, 1, 1, 128), (1, 20, 4, 8192, 128, 1, 1, 128),
             (2, 32, 8, 8192, 128, 1, 1, 128), (2, 32, 8, 16384, 128, 1, 1, 128),
             (4, 32, 8, 16384, 128, 1, 1, 128), (1, 64, 16, 16384, 128, 1, 1, 128)]
    shapes = [s + t + (st,) for s in fixed for t in TOPOLOGIES for st in (0, 1)]
    rng = np.random.default_rng(seed)
    while len(shapes) < count:
        B = int(rng.integers(1, 7))
        hkv = int(rng.integers(1, 17))
        group = int(rng.choice([1, 2, 3, 4, 5, 7, 8]))
        hq = hkv * group
        d = int(rng.choice([16, 32, 64, 128]))
        bm = 128 if rng.random() < 0.6 else int(rng.choice([32, 64, 96, 112, 120, 126, 160, 256]))
        pack = group if (group > 1 and bm % group == 0 and rng.random() < 0.5) else 1
        causal = int(rng.random() < 0.75)
        cus, xcds = TOPOLOGIES[int(rng.integers(len(TOPOLOGIES)))]
        max_n = max(1, 40000 * bm // max(1, B * (hq // pack) * pack))
        n = int(rng.integers(1, min(max_n, 20000) + 1))
        shapes.append((B, hq, hkv, n, d, causal, pack, bm, cus, xcds, int(rng.random() < 0.2)))
    return shapes


def restated(shape, plant=None, private_pct=sch.TAIL_PRIVATE_PCT):
    B, hq, hkv, n, d, causal, pack, bm, cus, xcds, static = shape
    plan, progs, tail_blocks = sch.launch_programs(B, hq, hkv, n, d, bool(causal), pack, bm, cus,
                                                   xcds, private_pct=private_pct, plant=plant)
    if static:
        plan.update(static_blocks=0, tail_wgs=0, queues=1, private=0, shared=0)
        tail_blocks = tail_blocks[:0]
    return plan, progs, tail_blocks


@pytest.fixture(scope="module")
def shapes():
    return sweep_shapes()


@needs_ablate
@pytest.mark.parametrize("private_pct", [-1, 50, 100])
def test_library_map_runs_every_program_once_and_equals_the_restatement(shapes, private_pct):
    """-1: the shipped policy (one shared pool); 50 and 100: per-XCD queues as variant builds
    plan them (FA2_TAIL_PRIVATE_PCT), the kernel's queue rules included."""
    fn = _map_fn()
    pct = sch.TAIL_PRIVATE_PCT if private_pct < 0 else private_pct
    tails = fallback_tails = queued = 0
    for i, shape in enumerate(shapes):
        B, hq, hkv, n, d, causal, pack, bm, cus, xcds, static = shape
        got, info = library_map(fn, shape, seed=i, private_pct=private_pct)
        plan, progs, tail_blocks = restated(shape, private_pct=pct)
        # the plan: grid decomposition, unit chunk, topology and tail policy
        for key in ("n_tiles", "n_bh", "unit_chunk", "xcd_shift", "tail_wgs", "queues", "private",
                    "shared"):
            assert info[key] == plan[key], (shape, key, info[key], plan[key])
        assert info["nonzero_words"] == 0, shape  # every ticket word wrapped back to zero
        programs = plan["grid"]
        if plan["tail_wgs"]:
            tails += 1
            fallback_tails += plan["queues"] == 1
            queued += plan["queues"] > 1
            s0 = plan["static_blocks"]
            assert info["static_blocks"] == s0 and info["grid"] == s0 + plan["tail_wgs"], shape
            assert s0 + len(tail_blocks) == programs, shape
            # the static part, workgroup for workgroup
            assert np.array_equal(got[:s0], progs[:s0]), shape
            # the tail: the programs of the tail's blocks, in any order; the spares run nothing
            tail = got[s0:]
            ran = tail[tail[:, 0] >= 0]
            spare = tail[tail[:, 0] < 0]
            assert (spare == -1).all(), shape
            assert len(ran) == len(tail_blocks) and len(spare) == plan["tail_wgs"] - len(tail_blocks)
            want = progs[tail_blocks]
            assert np.array_equal(np.unique(ran, axis=0), np.unique(want, axis=0)), shape
            run = np.concatenate([got[:s0], ran])
        else:
            assert info["grid"] == programs, shape
            assert np.array_equal(got, progs), shape
            run = got
        errs = sch.coverage_errors(run, B, hq, pack, plan["n_tiles"])
        assert errs == [], (shape, errs)
    # the sweep reached tails of every kind (per-XCD queues where the policy has them, and the
    # shared pool alone)
    assert tails > 200 and fallback_tails > 50, (tails, fallback_tails)
    assert (queued > 50) == (pct > 0), (queued, pct)


@pytest.mark.parametrize("plant", ["chunk", "reverse", "tail"])
def test_planted_mistakes_fail_the_coverage_check(shapes, plant):
    """The exactly-once check must see an off-by-one in the unit chunk, the reversed second round
    or the tail's private blocks (per-XCD queues, as a 50% build plans them): each planted in
    the restatement fails on the sweep."""
    failed = {True: 0, False: 0}   # by order: XCD-aware (units split over the XCDs) or fallback
    for shape in shapes:
        B, hq, hkv, n, d, causal, pack, bm, cus, xcds, static = shape
        plan, progs, tail_blocks = restated(shape, plant=plant, private_pct=50)
        if plan["tail_wgs"]:
            run = np.concatenate([progs[:plan["static_blocks"]], progs[tail_blocks]])
        else:
            run = progs
        if sch.coverage_errors(run, B, hq, pack, plan["n_tiles"]):
            failed[(B * hkv) % (1 << plan["xcd_shift"]) == 0] += 1
    assert failed[True] > 0, plant
    if plant == "reverse":   # the reversed second slots exist in both orders
        assert failed[False] > 0, plant


@needs_ablate
@pytest.mark.parametrize("shape", [(1, 32, 8, 2048, 128, 1, 1, 128), (2, 16, 16, 2048, 128, 1, 1, 128),
                                   (4, 16, 16, 1024, 128, 1, 1, 128), (1, 32, 8, 2048, 64, 1, 1, 128)])
def test_one_round_causal_grids_pair_heavy_with_light(shape):
    """What the reversed second slots are for: on a causal grid of at most two programs per CU,
    the two workgroups that meet on one CU (blocks b and b + 256 on MI355X) run q tiles t and
    n_tiles - 1 - t, so every CU gets the same number of key tiles (XCD-aware order: the units
    split over the 8 XCDs)."""
    fn = _map_fn()
    got, info = library_map(fn, shape + (256, 8, 0))
    assert info["tail_wgs"] == 0 and info["grid"] <= 512, info
    n_tiles = info["n_tiles"]
    first, second = got[:256, 0], got[256:info["grid"], 0]
    assert (first[: len(second)] + second == n_tiles - 1).all(), shape


def test_restatement_is_exact_without_plants(shapes):
    for shape in shapes[:400]:
        B, hq, hkv, n, d, causal, pack, bm, cus, xcds, static = shape
        plan, progs, tail_blocks = restated(shape)
        run = np.concatenate([progs[:plan["static_blocks"]], progs[tail_blocks]]) if plan["tail_wgs"] else progs
        assert sch.coverage_errors(run, B, hq, pack, plan["n_tiles"]) == [], shape


@needs_ablate
def test_topology_rules():
    """The device's (CUs, XCDs) -> the order's XCD count: powers of two up to 16 that divide the
    CUs; anything else is ordered as one XCD. Read back through the map's plan."""
    fn = _map_fn()
    for (cus, xcds), shift in {(256, 8): 3, (304, 8): 3, (32, 1): 0, (128, 4): 2, (64, 2): 1,
                               (228, 6): 0, (256, 32): 0, (100, 8): 0, (256, 16): 4}.items():
        _, info = library_map(fn, (1, 32, 8, 1024, 128, 1, 1, 128, cus, xcds, 0))
        assert info["xcd_shift"] == shift == sch.make_topology(cus, xcds)[0], (cus, xcds)
    # C3 on MI355X keeps the tuned order: XCD-aware, a tail of 64 programs per XCD in one shared
    # pool; a build with half of them private gives each XCD a queue of 32
    _, info = library_map(fn, (1, 32, 8, 8192, 128, 1, 1, 128, 256, 8, 0))
    assert (info["static_blocks"], info["tail_wgs"], info["queues"], info["private"],
            info["shared"]) == (1536, 640, 1, 0, 512)
    _, info = library_map(fn, (1, 32, 8, 8192, 128, 1, 1, 128, 256, 8, 0), private_pct=50)
    assert (info["static_blocks"], info["tail_wgs"], info["queues"], info["private"],
            info["shared"]) == (1536, 640, 8, 32, 256)
