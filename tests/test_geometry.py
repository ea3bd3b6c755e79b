"""CPU replay of the fused GEMV kernel's work mapping (no GPU).

Restates, step by step, the host-side launch sizing of `launch_gemv` and the device-side item walk of `gemv_kernel`
(paia-project_amd/csrc/gemv_kernel.h) and checks, for every variant knob combination and for awkward and real shapes:
  * every weight chunk of every row is consumed exactly once (so every byte of W is read once),
  * every output row is stored exactly once,
  * split-K (H=1): every wave of a block reaches the same number of barriers, and LDS partial slots stay in range,
  * the LDS request fits (x staging + INT4 sums + split-K partials <= 64 KiB); K beyond that runs the
    x-from-global launch (launch_gemv_xg: split-K, R=1, U=2, W=8, only the partials in LDS), replayed the same way.
This is the gfx950 counterpart of the reference's index-logic replay (src/tests/emulate_mapping.py:10-66), re-derived
for the wave64 item geometry. The constants below are the kernel's (kChunkBytes, kPartBytes, kMaxLds, FmtInfo::kXQ).
"""
import itertools
import math

import pytest

CHUNK = 1024        # bytes one wave reads from a row with one 16-byte load per lane
PART_BYTES = 8192   # LDS reserved for split-K partials
MAX_LDS = 65536
XQ = {"bf16": 1, "fp8": 2, "int4": 4, "int4zp": 4}


def row_bytes(fmt, K):
    return {"bf16": 2 * K, "fp8": K}.get(fmt, K // 2)


def lds_bytes(fmt, nchunks):
    x = nchunks * XQ[fmt] * CHUNK
    s32 = nchunks * 64 * 4 if fmt.startswith("int4") else 0
    return x + s32


def lds_plan(fmt, nchunks, R, W, H):
    """gemv_lds_plan: (LDS bytes, groups per combine round), or (0, 1) when K is too large. INT4 adds 16 bytes of
    per-wave window flags and one |x|-maximum slot per wave, rounded to 16 bytes (lds_slot_bytes)."""
    base = lds_bytes(fmt, nchunks) + ((16 + W * 4 + 15) // 16 * 16 if fmt.startswith("int4") else 0)
    if base > MAX_LDS:
        return 0, 1
    if not H:
        return base, 1
    gb = W * R * 4
    part = min(MAX_LDS - base, PART_BYTES)
    part -= part % gb
    if part < gb:
        return 0, 1
    return base + part, part // gb


def busiest_cu(ng, grid, W, cus):
    """Row groups of the busiest CU, counted group by group: block b (on CU b mod cus), wave w takes groups
    b*W + w + k*grid*W."""
    load = [0] * cus
    for g in range(ng):
        load[(g % (grid * W)) // W % cus] += 1
    return max(load)


XG_KNOBS = (1, 2, 8, 1)   # launch_gemv_xg: R, U, W, H


def launch(fmt, N, K, R, U, W, H, cus, per_cu):
    """Host sizing (launch_gemv): the params the kernel sees. p["knobs"] are the (R, U, W, H) that run: the call's,
    or launch_gemv_xg's when the staged x does not fit the LDS (p["xg"])."""
    rb = row_bytes(fmt, K)
    nchunks = -(-rb // CHUNK)
    lds, rnd = lds_plan(fmt, nchunks, R, W, H)
    xg = lds == 0
    if xg:
        R, U, W, H = XG_KNOBS
        lds = PART_BYTES
        rnd = PART_BYTES // (W * R * 4)
        per_cu = min(per_cu, 4)      # 8-wave blocks: at most 32 waves per CU
    p = {"N": N, "rb": rb, "nchunks": nchunks, "nseg": -(-nchunks // U), "ngroups": -(-N // R), "xg": xg,
         "knobs": (R, U, W, H)}
    per_cu = min(per_cu, max(1, (160 * 1024) // lds))
    if W >= 16:
        per_cu = 1                   # a 16-wave block runs alone on its CU
    if H and p["nseg"] == 1 and fmt == "bf16" and not xg:
        per_cu = min(per_cu, 2)      # BF16, one segment per row: one streaming wave per block, 2 blocks per CU
    gmax = cus * per_cu
    unit = 1 if H else W
    ng = p["ngroups"]
    grid = min(-(-ng // unit), gmax)
    q = -(-ng // (grid * unit))
    if not H:
        q = min(q, 64 // R)          # epilogue operands of all of a wave's groups in one register
    grid = -(-ng // (q * unit))
    if not H and per_cu >= 2 and q >= 2:
        # a whole number of blocks per CU when that lowers the busiest CU's groups
        b = min(-(-(-(-ng // cus)) // (q * W)), per_cu)
        if -(-ng // (cus * b * W)) <= q and busiest_cu(ng, cus * b, W, cus) < busiest_cu(ng, grid, W, cus):
            grid = cus * b
    p["grid"] = grid
    p["round"] = rnd
    return p


def walk(p, block, wave, R, U, W, H):
    """The items of one wave in order: (group, chunk0, slot, last), as ItemWalker/issue produce them."""
    if H:
        g, gstride, s0, sstep = block, p["grid"], wave, W
    else:
        g, gstride, s0, sstep = block * W + wave, p["grid"] * W, 0, 1
    s, k = s0, 0
    while g < p["ngroups"] and s0 < p["nseg"]:
        yield g, s * U, k % p["round"], s + sstep >= p["nseg"], k
        s += sstep
        if s >= p["nseg"]:
            s, g, k = s0, g + gstride, k + 1


def replay(fmt, N, K, R, U, W, H, cus=256, per_cu=4):
    p = launch(fmt, N, K, R, U, W, H, cus, per_cu)
    R, U, W, H = p["knobs"]
    seen = {}                              # (group, chunk) -> count (chunks < nchunks only)
    stored = [0] * N
    for b in range(p["grid"]):
        ngb = (p["ngroups"] - 1 - b) // p["grid"] + 1 if b < p["ngroups"] else 0
        barriers = []
        parked = set()                     # (k, wave): partial sums written to LDS (H=1)
        for w in range(W):
            nbar = 0
            items = list(walk(p, b, w, R, U, W, H))
            finished = 0
            for g, c0, slot, last, k in items:
                assert 0 <= slot < p["round"]
                assert (slot * W + w) * R + R <= p["round"] * W * R or not H
                for c in range(c0, c0 + U):
                    if c * CHUNK < p["rb"]:
                        seen[(g, c)] = seen.get((g, c), 0) + 1
                    # x index clamp keeps LDS reads in range (the x-from-global launch reads x bounded to K)
                    assert p["xg"] or min(c, p["nchunks"] - 1) * XQ[fmt] * CHUNK < lds_bytes(fmt, p["nchunks"])
                if last:
                    finished += 1
                    if not H:
                        # the store lanes k*R + r hold the group's epilogue operands: k must fit one register
                        assert k < 64 // R, f"wave group index {k} beyond the epilogue register (R={R})"
                        for r in range(R):
                            if g * R + r < N:
                                stored[g * R + r] += 1
                    else:
                        parked.add((k, w))
                        k_cur = k + 1
                        if slot == p["round"] - 1 or k_cur == ngb:
                            nbar += 2
            if H and not items:
                nbar = 2 * math.ceil(ngb / p["round"]) if ngb else 0
            barriers.append(nbar)
        if H:
            assert len(set(barriers)) == 1, f"block {b}: waves reach different barrier counts {barriers}"
            # the combine reads the partials of waves 0 .. min(W, nseg)-1 for every group: all must have been written
            reads = {(k, w) for k in range(ngb) for w in range(min(W, p["nseg"]))}
            assert reads == parked, f"block {b}: combine reads unwritten partials {sorted(reads - parked)[:4]}"
            for k in range(ngb):
                g = b + k * p["grid"]
                for r in range(R):
                    if g * R + r < N:
                        stored[g * R + r] += 1
    assert all(v == 1 for v in seen.values()), "a chunk was consumed twice"
    want = {(g, c) for g in range(p["ngroups"]) for c in range(p["nchunks"])}
    assert set(seen) == want, f"missing chunks: {sorted(want - set(seen))[:5]}"
    assert all(v == 1 for v in stored), f"rows stored != once: {[i for i, v in enumerate(stored) if v != 1][:5]}"
    return p


KNOBS = {
    "bf16": list(itertools.product([1, 2, 4], [1, 2, 4, 8], [4, 8], [0, 1])),
    "fp8": list(itertools.product([1, 2, 4], [1, 2, 4], [4, 8], [0, 1])),
    "int4": list(itertools.product([1, 2, 4, 8], [1, 2, 4], [4, 8], [0, 1])),
}
W16 = [(R, U, 16, 0) for R in (1, 2) for U in (1, 2, 4)]   # one 16-wave block per CU, row-parallel only
for _f in ("fp8", "int4"):
    KNOBS[_f] = KNOBS[_f] + W16
# block sizes for whole blocks per CU on the small shapes (row-parallel only)
KNOBS["fp8"] += [(1, 2, 6, 0), (1, 2, 12, 0)]
KNOBS["int4"] += [(1, 1, 9, 0), (2, 1, 9, 0), (1, 1, 12, 0), (1, 1, 14, 0)]
KNOBS["int4zp"] = KNOBS["int4"]
SHAPES = {
    "bf16": [(1, 8), (3, 264), (7, 520), (33, 1032), (129, 4104), (257, 3584), (100, 18944), (65, 4096), (17, 14336)],
    "fp8": [(1, 16), (3, 528), (33, 1552), (257, 3584), (100, 18944), (65, 4096), (17, 14336)],
    "int4": [(1, 128), (3, 384), (33, 2176), (257, 3584), (100, 18944), (65, 4096), (17, 14336)],
}
SHAPES["int4zp"] = SHAPES["int4"]


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "int4", "int4zp"])
def test_every_chunk_once_every_row_once(fmt):
    for (R, U, W, H), (N, K) in itertools.product(KNOBS[fmt], SHAPES[fmt]):
        for cus, per_cu in ((4, 2), (256, 4)):
            replay(fmt, N, K, R, U, W, H, cus, per_cu)


def test_real_shapes_grid_and_lds():
    """Real BASELINE shapes on 256 CUs: the walk covers W exactly; x is staged in the LDS (no fallback) for every
    format."""
    shapes = [(6144, 4096), (4096, 4096), (4096, 14336), (3584, 3584), (3584, 18944), (4608, 3584)]
    for fmt, (N, K) in itertools.product(["bf16", "fp8", "int4zp"], shapes):
        for R, U, W, H in [(2, 2, 4, 0), (1, 4, 8, 1), (4, 1, 4, 0)]:
            if (R, U) not in {(r, u) for r, u, _, _ in KNOBS[fmt]}:
                continue
            assert not replay(fmt, N, K, R, U, W, H, 256, 4)["xg"]


def test_lds_limit_and_the_x_from_global_launch():
    """x is staged up to the documented maxima; beyond them (and, for split-K, where one round of partials no longer
    fits beside x) the launch runs the x-from-global kernel, whose walk covers every chunk and row once."""
    assert not launch("bf16", 8, 32768, 1, 1, 4, 0, 256, 1)["xg"]
    assert launch("bf16", 8, 32776, 1, 1, 4, 0, 256, 1)["xg"]
    assert launch("bf16", 8, 32768, 1, 1, 4, 1, 256, 1)["xg"]          # split-K needs room for one partial round
    assert not launch("bf16", 8, 32256, 4, 1, 8, 1, 256, 1)["xg"]
    assert not launch("fp8", 8, 32768, 1, 1, 4, 0, 256, 1)["xg"]
    assert not launch("int4", 8, 30720, 1, 1, 4, 0, 256, 1)["xg"]
    assert launch("int4", 8, 30848, 1, 1, 4, 0, 256, 1)["xg"]
    for fmt, N, K in [("bf16", 33, 40000), ("bf16", 1, 65536 + 8), ("fp8", 129, 32784), ("fp8", 7, 100000),
                      ("int4", 65, 30848), ("int4zp", 3, 65536 + 128)]:
        for cus, per_cu in ((4, 2), (256, 4)):
            assert replay(fmt, N, K, 2, 2, 4, 0, cus, per_cu)["xg"]


def test_whole_blocks_per_cu_when_the_last_round_is_uneven():
    """H=0 over several rounds and blocks per CU: the grid is a whole number of blocks per CU exactly when that lowers
    the busiest CU's row groups (counted group by group), and never raises it or the rounds per wave."""
    cases = {(14336, 8, 4): 1024, (18944, 8, 4): 1024, (10112, 8, 4): 768, (10368, 8, 4): 648, (9472, 4, 8): 1184,
             (14336, 4, 8): 1792, (2048, 4, 8): 512}   # (groups, W, blocks per CU) -> grid on 256 CUs
    for (ng, W, per_cu), want in cases.items():
        p = launch("fp8", ng, 4096, 1, 1, W, 0, 256, per_cu)
        assert p["grid"] == want, (ng, W, per_cu, p["grid"])
    for ng, W, per_cu in itertools.product([300, 1000, 2049, 6000, 9999, 14336, 40000], [4, 8], [2, 4, 8]):
        gmax = 256 * per_cu
        q = min(-(-ng // (min(-(-ng // W), gmax) * W)), 64)
        fewest = -(-ng // (q * W))
        p = launch("fp8", ng, 4096, 1, 1, W, 0, 256, per_cu)
        assert -(-ng // (p["grid"] * W)) <= q
        assert busiest_cu(ng, p["grid"], W, 256) <= busiest_cu(ng, fewest, W, 256)


def test_groups_per_wave_capped_for_the_epilogue_register():
    """Tall N on a small grid: without the cap a wave would own more than 64/R groups (its epilogue operands would
    not fit the one register loaded before the streaming loop); the launch grows the grid instead."""
    for R, U, W in [(1, 1, 4), (2, 2, 4), (4, 1, 8), (8, 1, 4)]:
        replay("fp8", 40000, 256, R, U, W, 0, cus=2, per_cu=1)


def test_one_segment_split_k_runs_two_blocks_per_cu():
    """BF16 split-K with rows one segment long (the lm_heads at U = 8): one wave per block streams, the launch holds
    at most 2 blocks per CU, and the walk still covers every row once. Other formats keep the general sizing."""
    for N, K in [(128256, 4096), (152064, 3584)]:
        p = launch("bf16", N, K, 2, 8, 8, 1, 256, 4)
        assert p["nseg"] == 1 and p["grid"] <= 2 * 256
        replay("bf16", N // 64, K, 2, 8, 8, 1, 256, 4)     # coverage on a smaller N with the same walk
    assert launch("bf16", 128256, 4096, 2, 4, 8, 1, 256, 4)["grid"] > 2 * 256   # two segments: unchanged
    assert launch("fp8", 128256, 4096, 1, 4, 4, 1, 256, 8)["grid"] > 2 * 256    # FP8: general sizing
