"""Launch geometry of the small-row matmul (libnmx.so nmx_mt_plan; no GPU needed).

The kernel (nibblemac_amd/csrc/hip/nmx_mt.hip, q4k_mt_k) runs phases whose work items are
dealt to threads one each: weight units, (row, vector) chains, the norm prologue's columns,
its per-row chains and tails, the MTP fc input's h float4s and embedding blocks, the SwiGLU
epilogue's output columns. A phase with more work items than threads leaves LDS unwritten that
a later phase reads (the stale-norm bug once fixed in the MTP fc prologue, where the thread
count came from the weight units alone). Here every shape the engine's loader admits is
planned on the host and each phase's need is restated from the kernel's structure, so a
planner change that starves a phase fails on the CPU before any launch. The launch itself
refuses such a geometry (mt_geometry_error).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "nibblemac_amd" / "lib" / "libnmx.so"
LDS_MAX = 159 * 1024
MAX_NV = 8


class Geometry(ctypes.Structure):
    _fields_ = [("rows_per_wg", ctypes.c_int), ("threads", ctypes.c_int),
                ("blocks_per_unit", ctypes.c_int), ("workgroups", ctypes.c_int),
                ("passes", ctypes.c_int), ("nv", ctypes.c_int * 8),
                ("lds_bytes", ctypes.c_int * 8)]


@pytest.fixture(scope="module")
def plan():
    if not LIB.exists():
        pytest.skip("libnmx.so not built")
    lib = ctypes.CDLL(str(LIB))
    f = lib.nmx_mt_plan
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int,
                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Geometry)]

    def run(rows, cols, n, norm=False, swiglu=False, pair=False):
        arr = (ctypes.c_int * len(rows))(*rows)
        g = Geometry()
        rc = f(len(rows), arr, cols, n, int(norm), int(swiglu), int(pair), ctypes.byref(g))
        return rc, g
    return run


def bound(norm, swiglu, bpu):
    """__launch_bounds__ of q4k_mt_k for the variant."""
    return 1024 if bpu < 4 else 512 if norm else 512 if swiglu else 256


def needs(cols, nv, R, bpu, norm, swiglu, pair):
    """Threads each phase of q4k_mt_k needs, one work item per thread."""
    nsb = cols // 256
    out = {"weight units": R * (8 // bpu) * nsb, "chains": R * nv}
    if norm and not pair:
        cpt = 2 if bpu < 4 else 8  # columns per thread of the plain prologue
        out["norm columns"] = -(-cols // cpt)
    if norm:
        out["norm chains and tails"] = 5 * (2 if pair else 1) * nv
    if pair:
        out["h float4s"] = cols // 8             # cols / 2 columns of h, one float4 each
        out["embedding blocks"] = nv * (cols // 64)  # nv rows x (cols / 2) / 32 blocks
    if swiglu:
        out["SwiGLU outputs"] = nv * (R // 2)
    return out


def lds_floor(cols, nv, R, swiglu):
    """Bytes the phases store in LDS at least: the A8 codes and (d, fsum) of the pass, and the
    chain records (16 bytes per (block, vector, row); SwiGLU 8 + 4 per (block, row))."""
    nb = cols // 32
    rec = nb * nv * R * 8 + nb * R * 4 if swiglu else nb * nv * R * 16
    return nb * nv * 32 + nb * nv * 8 + rec


def check(plan, rows, cols, n, norm=False, swiglu=False, pair=False):
    rc, g = plan(rows, cols, n, norm, swiglu, pair)
    if rc == 0:
        return False
    assert rc == 1, f"planner picked a geometry the launch refuses: {rows} {cols} {n}"
    R, T, bpu = g.rows_per_wg, g.threads, g.blocks_per_unit
    assert T % 64 == 0 and 64 <= T <= bound(norm, swiglu, bpu), (T, bpu)
    assert R >= 4 and R % 4 == 0
    assert bpu in (1, 2, 4) and (not pair or bpu == 1)
    if swiglu:
        assert R == 64
    # equal passes of at most 8 vectors, larger first, covering n
    nvs = list(g.nv[:g.passes])
    assert sum(nvs) == n and max(nvs) <= MAX_NV and nvs == sorted(nvs, reverse=True)
    assert max(nvs) - min(nvs) <= 1 and g.passes == -(-n // MAX_NV)
    for p, nv in enumerate(nvs):
        for phase, need in needs(cols, nv, R, bpu, norm, swiglu, pair).items():
            assert T >= need, f"{phase}: {need} items, {T} threads ({rows} {cols} n={n} nv={nv})"
        assert lds_floor(cols, nv, R, swiglu) <= g.lds_bytes[p] <= LDS_MAX
    wg = rows[0] // (R // 2) if swiglu else sum(-(-r // R) for r in rows)
    assert g.workgroups == wg
    return True


COLS = list(range(256, 16384 + 1, 256)) + [20480, 32768, 65536]


@pytest.mark.parametrize("n", range(1, MAX_NV + 1))
def test_norm_prologue_geometry(plan, n):
    """The input projections with the block's RMSNorm inside: one to four matrices over the
    hidden size (the DeltaNet qkv/z/b/a and the attention q/k/v groups among them)."""
    taken = 0
    for H in COLS:
        for rows in ([H], [2 * H, H], [H, 256, 256], [3 * H, H, 32, 32], [4, 4], [8192, 28],
                     [H // 4, H // 4, H // 4]):
            rows = [r for r in rows if r > 0]
            if sum(rows) >= 32768:
                continue
            taken += check(plan, rows, H, n, norm=True)
    assert taken > 40


@pytest.mark.parametrize("n", range(1, MAX_NV + 1))
def test_swiglu_geometry(plan, n):
    """Gate and up (ffn rows each, over the hidden size) with the post-mixer norm inside or
    plain A8 inputs, and the SiLU-product + A8 epilogue."""
    taken = 0
    for H in COLS:
        for ffn in (256, 512, 1024, 3584, 4096, 8192, 16128):
            for norm in (False, True):
                taken += check(plan, [ffn, ffn], H, n, norm=norm, swiglu=True)
    assert taken > 40


@pytest.mark.parametrize("n", range(1, MAX_NV + 1))
def test_mtp_fc_pair_geometry(plan, n):
    """The MTP fc projection (H rows over [embedding | hidden], 2 H columns) with the
    embedding row's decode and both input norms inside."""
    taken = sum(check(plan, [H], 2 * H, n, norm=True, pair=True) for H in COLS if H < 32768)
    assert taken >= 3


@pytest.mark.parametrize("n", range(1, MAX_NV + 1))
def test_plain_projection_geometry(plan, n):
    """The projections without a prologue (out, o, down): H rows over the mixer or FFN
    width, and multi-matrix groups."""
    taken = 0
    for cols in COLS:
        for rows in ([1024], [256], [4], [4096, 4096], [8192, 1024, 16, 16], [16384]):
            taken += check(plan, rows, cols, n)
    assert taken > 100


def test_verify_shapes_are_fused(plan):
    """The 0.8B-shape verify pass (hidden 1024, FFN 3584, k + 1 = 5 rows) runs every one of
    these projections in the fused kernel, so the checks above cover the shapes the bench runs."""
    for rows, cols, kw in [([6144, 2048, 16, 16], 1024, {"norm": True}),
                           ([2048, 512, 512], 1024, {"norm": True}),
                           ([3584, 3584], 1024, {"norm": True, "swiglu": True}),
                           ([1024], 2048, {}), ([1024], 3584, {}),
                           ([1024], 2048, {"norm": True, "pair": True})]:
        for n in (1, 5):
            assert check(plan, rows, cols, n, **kw), (rows, cols, n, kw)


def test_pair_planner_refuses_misaligned_shapes(plan):
    """PAIR halves must be whole superblocks (cols a multiple of 512); otherwise the shape goes
    to the separate norm + matmul."""
    assert plan([256], 768, 1, True, False, True)[0] == 0
    assert plan([256], 1024, 9, True, False, True)[0] == 0  # more than 8 vectors
