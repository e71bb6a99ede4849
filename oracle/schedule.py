"""CPU restatement of the forward launch's program order: TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/ may import this module, as the checker of the library's own schedule code
(fa2_ablate_program_map runs the kernel's program_of and tail rules on the CPU). The product path
never calls into it.

The reference launches one program per (q tile, batch x head group) and computes each alone
(fa2/kernel.py:24-26, 126-132), so the order of programs never changes a result; what must hold
is that every program runs exactly once. This module restates, in numpy over whole launches, the
HIP build's order (csrc/attn_fwd_schedule.hpp) and host policy (csrc/attn_fwd_host.hpp):

  make_topology    the device's (CUs, XCDs) -> (log2 XCDs, CUs) the order uses
  unit_chunk       units per chunk of an XCD's causal q-tile-major order
  tail_schedule    the dynamic tail: static blocks, tail workgroups, queues, private / shared
  program_of       block -> (q tile, batch, first query head), vectorised over blocks
  launch_programs  every program of a launch in block order (the static order)
  coverage_errors  the exactly-once check: what is wrong with a list of run programs

How each is pinned (tests/test_schedule.py): the library's map must equal this restatement
workgroup for workgroup on the static part and as a set on the tail, over thousands of launch
shapes and several topologies; coverage_errors must find nothing in the library's map; and
planted mistakes in this restatement (an off-by-one in the chunk, the reversed second round or
the tail's private blocks) must make coverage_errors fail on the same sweep, so the check is able
to see such a mistake.
"""

import numpy as np

KCUS, KXCDS, KMAX_XCDS = 256, 8, 16
CHUNK_KV_BYTES = 8 << 20
TAIL_PRIVATE_PCT = 0   # the shipped policy; builds can differ (FA2_TAIL_PRIVATE_PCT)
XCD_REVERSE = True     # the shipped order; builds can differ (FA2_XCD_REVERSE)


def make_topology(cus, xcds):
    """(xcd_shift, cus): a power-of-two XCD count up to 16 that divides the CUs, else one XCD."""
    cus = cus if cus > 0 else KCUS
    shift = 0
    if 1 < xcds <= KMAX_XCDS and xcds & (xcds - 1) == 0 and cus % xcds == 0:
        while (1 << shift) < xcds:
            shift += 1
    return shift, cus


def unit_chunk(units, n_kv, head_dim, topo):
    upx = units >> topo[0]
    if upx < 1:
        return 1
    unit_kv = 4 * n_kv * head_dim
    chunk = max(1, CHUNK_KV_BYTES // unit_kv) if unit_kv > 0 else upx
    if chunk >= upx:
        return upx
    while upx % chunk:
        chunk -= 1
    return chunk


def tail_schedule(causal, waves, units, progs_per_kv, n_tiles, chunk, head_dim, bn, topo,
                  private_pct=TAIL_PRIVATE_PCT):
    """dict(static_blocks, tail_wgs, queues, private, shared); tail_wgs 0 = the static order."""
    none = dict(static_blocks=0, tail_wgs=0, queues=1, private=0, shared=0)
    if not causal or waves != 4:
        return none
    xcds = 1 << topo[0]
    slots = max(1, topo[1] // xcds) * (3 if (head_dim == 64 and bn <= 64) else 2)
    grid = units * progs_per_kv * n_tiles
    extra = (grid * 6 // 100 + xcds - 1) // xcds * xcds
    if grid + extra > 0x7FFFFFFF:
        return none
    if units % xcds:
        per_xcd = grid // xcds
        if per_xcd < 2 * slots:
            return none
        static = (per_xcd - (per_xcd + 3) // 4) * xcds
        return dict(static_blocks=static, tail_wgs=grid - static + extra, queues=1, private=0,
                    shared=grid - static)
    upx = units // xcds
    per_xcd = upx * progs_per_kv * n_tiles
    if per_xcd < 2 * slots:
        return none
    cu = chunk if (chunk > 0 and upx % chunk == 0) else upx
    tail = min((per_xcd + 3) // 4, cu * progs_per_kv * n_tiles // 2)
    if tail < 1:
        return none
    priv = tail * private_pct // 100
    queues = xcds if (xcds > 1 and priv > 0) else 1
    private = priv if queues > 1 else 0
    return dict(static_blocks=(per_xcd - tail) * xcds, tail_wgs=tail * xcds + extra,
                queues=queues, private=private, shared=tail * xcds - queues * private)


def program_of(blocks, *, causal, h_q, group, pack, n_tiles, n_bh, unit_chunk, xcd_shift, cus,
               plant=None):
    """(tile, b, hq0) arrays for an int64 array of blocks. `plant` names a deliberate mistake
    (tests only): "chunk" or "reverse"."""
    blocks = np.asarray(blocks, dtype=np.int64).copy()
    ppk = group // pack
    h_kv = h_q // group
    units = n_bh // ppk
    xcds = 1 << xcd_shift
    if units % xcds == 0:
        xcd = blocks & (xcds - 1)
        slot = blocks >> xcd_shift
        upx = units >> xcd_shift
        if causal:
            cu = unit_chunk if (unit_chunk > 0 and upx % unit_chunk == 0) else upx
            per_chunk = cu * ppk * n_tiles
            cpx = cus >> xcd_shift
            per_xcd = upx * ppk * n_tiles
            if XCD_REVERSE and per_xcd <= 2 * cpx:
                sel = slot >= cpx
                back = cpx + (per_xcd - 1 - slot) if plant != "reverse" else cpx + (per_xcd - slot)
                slot = np.where(sel, back, slot)
            ch = slot // per_chunk
            rs = slot - ch * per_chunk
            per_t = cu * ppk
            t = rs // per_t
            r = rs - t * per_t
            kv = xcd * upx + ch * cu + r // ppk
            if plant == "chunk":
                kv = xcd * upx + ch * (cu - 1) + r // ppk
            h_in = r % ppk
        else:
            per_u = n_tiles * ppk
            u = slot // per_u
            r = slot - u * per_u
            t = r // ppk
            h_in = r - t * ppk
            kv = xcd * upx + u
    else:
        grid = n_tiles * n_bh
        if causal and grid <= 3 * cus:
            end = min(grid, 2 * cus)
            sel = (blocks >= cus) & (blocks < end)
            back = cus + (end - 1 - blocks) if plant != "reverse" else cus + (end - blocks)
            blocks = np.where(sel, back, blocks)
        t = blocks // n_bh
        r = blocks - t * n_bh
        kv = r // ppk
        h_in = r - kv * ppk
    tile = n_tiles - 1 - t if causal else t
    b = kv // h_kv
    hkv = kv - b * h_kv
    return tile, b, hkv * group + h_in * pack


def launch_programs(batch, h_q, h_kv, n_q, head_dim, causal, pack, block_m, cus, xcds,
                    private_pct=TAIL_PRIVATE_PCT, plant=None):
    """The restated launch: (dict of its plan, [P, 3] programs in block order of the static
    order, [T] blocks its dynamic tail deals, in ticket order: every private ticket of every queue,
    then every shared ticket). `plant` (tests only): "chunk", "reverse" or "tail"."""
    topo = make_topology(cus, xcds)
    group = h_q // h_kv
    waves = 1
    while waves * 32 < block_m:
        waves *= 2
    bn = 128 if head_dim == 16 else 64
    n_tiles = (n_q * pack + block_m - 1) // block_m
    n_bh = batch * (h_q // pack)
    ppk = group // pack
    units = n_bh // ppk
    chunk = unit_chunk(units, n_q, head_dim, topo)
    ts = tail_schedule(causal, waves, units, ppk, n_tiles, chunk, head_dim, bn, topo, private_pct)
    grid = n_tiles * n_bh
    tile, b, hq0 = program_of(np.arange(grid), causal=causal, h_q=h_q, group=group, pack=pack,
                              n_tiles=n_tiles, n_bh=n_bh, unit_chunk=chunk, xcd_shift=topo[0],
                              cus=topo[1], plant=plant if plant in ("chunk", "reverse") else None)
    progs = np.stack([tile, b, hq0], axis=1)
    tail_blocks = np.zeros(0, dtype=np.int64)
    if ts["tail_wgs"]:
        q, priv, s0 = ts["queues"], ts["private"], ts["static_blocks"]
        t = np.arange(priv)
        x = np.arange(q)
        stride = q + 1 if plant == "tail" else q
        private = (s0 + t[None, :] * stride + x[:, None]).reshape(-1)
        shared = s0 + q * priv + np.arange(ts["shared"])
        tail_blocks = np.concatenate([private, shared])
    plan = dict(ts, grid=grid, n_tiles=n_tiles, n_bh=n_bh, unit_chunk=chunk, xcd_shift=topo[0],
                cus=topo[1])
    return plan, progs, tail_blocks


def coverage_errors(run, batch, h_q, pack, n_tiles):
    """What is wrong with `run`, an [R, 3] array of the (tile, b, hq0) programs a launch ran
    (spare workgroups left out): [] when every program of the grid ran exactly once."""
    run = np.asarray(run, dtype=np.int64).reshape(-1, 3)
    errs = []
    tile, b, hq0 = run[:, 0], run[:, 1], run[:, 2]
    bad = (tile < 0) | (tile >= n_tiles) | (b < 0) | (b >= batch) | (hq0 < 0) | (hq0 >= h_q) | (hq0 % pack != 0)
    if bad.any():
        errs.append(f"{int(bad.sum())} programs outside the grid, e.g. {run[bad][0].tolist()}")
        return errs
    key = (tile * batch + b) * h_q + hq0
    uniq, counts = np.unique(key, return_counts=True)
    if (counts > 1).any():
        errs.append(f"{int((counts > 1).sum())} programs ran more than once")
    expected = n_tiles * batch * (h_q // pack)
    if uniq.size != expected:
        errs.append(f"{expected - uniq.size} of {expected} programs never ran")
    return errs
