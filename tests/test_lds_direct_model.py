"""Host model of every LDS-direct buffer load the library issues (buffer_load_dword ... lds, through
__builtin_amdgcn_raw_ptr_buffer_load_lds with 4 bytes per lane), bounds-checked on the CPU at every launch shape the
library accepts.

Semantics modelled (CDNA buffer instructions with the LDS bit): lane l of the wave reads the 4 bytes at
base + voffset(l) + soffset + inst_offset of the buffer resource (base, num_records) and writes them to LDS at
M0 + inst_offset + 4 l, where M0 is the wave-uniform LDS address the builtin takes; a read at or past num_records
returns zeros. The kernels pass inst_offset = 0. What must hold for every load of every lane:
  * the global read lies inside the buffer (voffset + soffset + 4 <= num_records), inside the matrix or input array
    it is meant to read, and every offset fits the 32-bit fields (num_records, voffset, soffset < 2^31);
  * the LDS write lies inside the wave's own ring slot (decode, grouped GEMM) or the workgroup's shared ring slot
    (chain GEMM, input rings), and the rings lie inside the dynamic LDS the launcher requests, itself <= 160 KB.

The kernels' constants are read from their sources, so the model follows the code. Streaming loops modelled:
chain_dma (decode, per-slot and per-expert launches) and chain_mf (decode mode MFMA), k_moe.hip; gp_gemm_kernel
(MFMA grouped GEMM) and xg_gemm_kernel (EXACT accumulator chains), k_prefill.hip. The relay launches stream through
registers (16-byte buffer loads) and are modelled too, for the same global bounds. Shapes: K = 2..5, H and I every
multiple of 256 from 256 to GFL_MAX_DIM (32768) on a grid that includes both ends, the configs' 5120 / 1536, and the
largest slot counts the prefill path accepts.
"""
import os
import re

import numpy as np
import pytest

from conftest import ROOT

CSRC = os.path.join(ROOT, "glm-flash-lite_amd", "csrc")
LDS_LIMIT = 163840
INT32_MAX = 2 ** 31 - 1


def _const(fname, name):
    text = open(os.path.join(CSRC, fname)).read()
    m = re.search(r"constexpr int %s = (\d+);" % name, text)
    assert m, (fname, name)
    return int(m.group(1))


def _max_dim():
    text = open(os.path.join(ROOT, "include", "gfl_moe.h")).read()
    return int(re.search(r"#define GFL_MAX_DIM (\d+)", text).group(1))


NGRP = _const("k_moe.hip", "NGRP")
GU_NW = _const("k_moe.hip", "GU_NW")
DN_NW = _const("k_moe.hip", "DN_NW")
GP_MT = _const("k_prefill.hip", "GP_MT")
GP_NW = _const("k_prefill.hip", "GP_NW")
GP_CPW = _const("k_prefill.hip", "GP_CPW")
GP_NG = _const("k_prefill.hip", "GP_NG")
GP_XS = _const("k_prefill.hip", "GP_XS")
XG_NW = _const("k_prefill.hip", "XG_NW")
XG_MS = _const("k_prefill.hip", "XG_MS")
XG_NG = _const("k_prefill.hip", "XG_NG")
XG_TC = 16 * XG_NW // 16
XG_XROW = 8 * 16 * 4
XG_XGB = XG_MS * XG_XROW
MAX_DIM = _max_dim()
MAX_GROUPED_PICKS = 65536

DIMS = sorted({256, 512, 768, 1024, 1536, 2048, 4096, 5120, 8192, 16384, 30464, MAX_DIM})
LANE = np.arange(64, dtype=np.int64)


def _check_global(voff, soff, nrec, lo, hi, what):
    """voff: int64 array of vector offsets, soff: scalar offsets (array broadcastable); every 4-byte read must lie in
    [lo, hi) relative to the resource base, inside num_records, with offsets in the 32-bit fields."""
    assert 0 < nrec <= INT32_MAX, (what, nrec)
    a = voff + soff
    assert voff.min() >= 0 and voff.max() <= INT32_MAX and np.min(soff) >= 0 and np.max(soff) <= INT32_MAX, what
    assert a.min() >= lo and a.max() + 4 <= hi, (what, int(a.min()), int(a.max()), lo, hi)
    assert a.max() + 4 <= nrec, (what, int(a.max()), nrec)
    assert (a % 4 == 0).all(), what


def _check_lds(dst, lo, hi, what):
    """dst: LDS byte offsets of each lane's 4-byte write; all inside [lo, hi)."""
    assert dst.min() >= lo and dst.max() + 4 <= hi, (what, int(dst.min()), int(dst.max()), lo, hi)


def _column_stream(K, kdim, ndim, t, NG, what, ring_lo, ring_hi):
    """chain_dma / chain_mf: the wave's tile column t of a [kdim/16][ndim/16] tile matrix, K dword loads per lane per
    group of 8 tile rows into ring slot g % NG of the wave's ring (k_moe.hip chain_dma: voff = (byte / TB) * gs +
    byte % TB with byte = 256 i + 4 lane, soffset = 8 g gs; buffer base = tile column t, num_records = TK * gs)."""
    TB, TK, TN = 32 * K, kdim // 16, ndim // 16
    GB, gs = 8 * TB, TN * TB
    i = np.arange(K, dtype=np.int64)[:, None]
    byte = i * 256 + 4 * LANE[None, :]
    voff = (byte // TB) * gs + byte % TB
    assert ((byte % TB) < TB).all() and ((byte // TB) < 8).all()
    g = np.arange(TK // 8, dtype=np.int64)
    soff = (8 * g * gs)[:, None, None]
    # relative to the resource base (tile column t of tile row 0): inside [0, TK * gs); absolutely, inside the matrix
    _check_global(voff[None], soff, TK * gs, 0, TK * gs, what)
    absolute = t * TB + voff[None] + soff
    assert absolute.max() + 4 <= TK * gs, what
    # the bytes read by the group's load i of lane l are tile row 8g + byte/TB of tile column t exactly
    assert (((absolute - t * TB) % gs) < TB).all(), what
    dst = (g[:, None, None] % NG) * GB + i[None] * 256 + 4 * LANE[None, None, :]
    _check_lds(ring_lo + dst, ring_lo, ring_hi, what)
    assert ring_hi - ring_lo == NG * GB, what


def _gu_lds(K, ns, H, P, E, mf):
    return GU_NW * NGRP * 8 * 32 * K + ns * H * (1 if mf else (4 if ns <= 1 else 2)) + (7 * P + 1 + 2 * E) * 4


def _dn_lds(K, ns, I, mf):
    nw = DN_NW // 2 if (ns == 1 and not mf) else DN_NW
    return nw * NGRP * 8 * 32 * K + ns * I * (2 if mf else (4 if ns <= 1 else 2)) + ns * 128 * 4, nw


@pytest.mark.parametrize("K", [2, 3, 4, 5])
def test_decode_streaming_loads_in_bounds(K):
    """gu_kernel / down_kernel (chain_dma, EXACT; chain_mf, mode MFMA) at every shape run_forward launches: the LDS
    request within 160 KB (else the call is refused before any launch) and every load of the first and last tile
    column of every matrix in bounds."""
    launched = 0
    for H in DIMS:
        for I in DIMS:
            for (ns, mf) in [(1, False), (2, False), (4, False), (8, False), (4, True)]:
                P, E = 1024, 1024
                gl = _gu_lds(K, ns, H, P, E, mf)
                dl, nw = _dn_lds(K, ns, I, mf)
                if gl > LDS_LIMIT or dl > LDS_LIMIT:
                    continue                     # run_forward refuses the shape (no launch)
                launched += 1
                for (kdim, ndim, nwaves) in [(H, I, GU_NW), (I, H, nw)]:
                    RB = NGRP * 8 * 32 * K
                    for t in (0, ndim // 16 - 1):
                        for w in (0, nwaves - 1):
                            _column_stream(K, kdim, ndim, t, NGRP, f"decode K={K} {kdim}x{ndim} ns={ns} mf={mf}",
                                           w * RB, (w + 1) * RB)
    assert launched > 0


def _relay_loads(K, kdim, ndim, t, RW, what):
    """chain_relay: 16-byte register loads, lane l of load i holds chunk q = 64 i + l of the group (tile q / 2K,
    bytes 16 (q % 2K) onward; lanes past the group read chunk 0), group index clamped to the last group."""
    TB, TK, TN = 32 * K, kdim // 16, ndim // 16
    CH, gs = 2 * K, TN * TB
    NCH = 8 * CH
    NLD = (NCH + 63) // 64
    q = 64 * np.arange(NLD, dtype=np.int64)[:, None] + LANE[None, :]
    voff = np.where(q < NCH, (q // CH) * gs + (q % CH) * 16, 0)
    ngroups = TK // 8
    g = np.minimum(np.arange(ngroups + 8, dtype=np.int64), ngroups - 1)
    soff = (8 * g * gs)[:, None, None]
    a = voff[None] + soff
    assert a.min() >= 0 and a.max() + 16 <= TK * gs <= INT32_MAX, what
    assert (t * TB + a).max() + 16 <= TK * gs, what


@pytest.mark.parametrize("K", [2, 3, 4, 5])
def test_relay_register_loads_in_bounds(K):
    for H in DIMS:
        for I in DIMS:
            for (kdim, ndim) in [(H, I), (I, H)]:
                for RW in (1, 2, 4):
                    for t in (0, ndim // 16 - 1):
                        _relay_loads(K, kdim, ndim, t, RW, f"relay K={K} {kdim}x{ndim} RW={RW}")


@pytest.mark.parametrize("K", [2, 3, 4, 5])
def test_grouped_gemm_loads_in_bounds(K):
    """gp_gemm_kernel: per wave a ring of GP_NG groups of 8 tile rows x GP_CPW tile columns (the wave's base at tile
    column t0), the slots' fp16 input chunks of 256 bytes through a shared ring of GP_MT rows of GP_XS fp16; slot rows
    past the pass repeat its last slot; inputs [cap][kdim] fp16 with cap * kdim * 2 <= 2^31 - 1 (gfl_grouped_forward
    refuses larger calls)."""
    TB = 32 * K
    RB, GB = GP_CPW * TB, 8 * GP_CPW * TB
    NLD = GB // 256
    assert GB % 256 == 0
    lds = GP_NW * GP_NG * GB + GP_NG * GP_MT * GP_XS * 2
    assert lds <= LDS_LIMIT
    xring0 = GP_NW * GP_NG * GB
    for kdim in DIMS:
        for ndim in DIMS:
            TK, TN = kdim // 16, ndim // 16
            gs = TN * TB
            if ndim % (16 * GP_NW * GP_CPW):
                continue
            for w in (0, GP_NW - 1):
                for t0 in (w * GP_CPW, TN - GP_CPW):
                    i = np.arange(NLD, dtype=np.int64)[:, None]
                    byte = i * 256 + 4 * LANE[None, :]
                    voff = (byte // RB) * gs + byte % RB
                    g = np.arange(TK // 8, dtype=np.int64)
                    soff = (8 * g * gs)[:, None, None]
                    what = f"gp_gemm K={K} {kdim}x{ndim} t0={t0}"
                    _check_global(voff[None], soff, TK * gs, 0, TK * gs, what)
                    assert (t0 * TB + voff[None] + soff).max() + 4 <= TK * gs, what
                    dst = w * GP_NG * GB + (g[:, None, None] % GP_NG) * GB + i[None] * 256 + 4 * LANE[None, None, :]
                    _check_lds(dst, w * GP_NG * GB, (w + 1) * GP_NG * GB, what)
            # the slots' inputs: cap up to the largest accepted call, rows of the pass's slots
            cap = min(MAX_GROUPED_PICKS, INT32_MAX // (kdim * 2))
            xpw = GP_MT // GP_NW
            slots = np.array([0, cap - 1], dtype=np.int64)
            g = np.arange(TK // 8, dtype=np.int64)
            voff = 4 * LANE
            soff = slots[:, None, None] * kdim * 2 + g[None, :, None] * 256
            _check_global(voff[None, None, :], soff, cap * kdim * 2, 0, cap * kdim * 2, f"gp_gemm x K={K} {kdim}")
            for w in (0, GP_NW - 1):
                for j in (0, xpw - 1):
                    for gg in (0, 1):
                        base = xring0 + (gg * GP_MT + w * xpw + j) * GP_XS * 2
                        _check_lds(base + 4 * LANE, xring0, lds, "gp_gemm x ring")
                        assert (4 * LANE).max() + 4 <= GP_XS * 2


@pytest.mark.parametrize("K", [2, 3, 4, 5])
def test_chain_gemm_loads_in_bounds(K):
    """xg_gemm_kernel: one shared ring of XG_NG groups of 8 tile rows x XG_TC tile columns (each wave loads its K
    dwords per lane of a group), the slots' fp32 inputs through a ring of XG_MS rows of 512 bytes per group; inputs
    [cap][kdim] fp32 with cap * kdim * 4 <= 2^31 - 1 (gfl_moe_forward refuses larger calls above 1,024 picks)."""
    TB = 32 * K
    RB, GB = XG_TC * TB, 8 * XG_TC * TB
    NLD = GB // 256 // XG_NW
    assert GB % (256 * XG_NW) == 0 and NLD == K
    lds = XG_NG * GB + XG_NG * XG_XGB
    assert lds <= LDS_LIMIT
    for kdim in DIMS:
        for ndim in DIMS:
            if ndim % (16 * XG_NW):
                continue
            TK, TN = kdim // 16, ndim // 16
            gs = TN * TB
            for nc in (0, TN // XG_TC - 1):
                for w in (0, XG_NW - 1):
                    i = np.arange(NLD, dtype=np.int64)[:, None]
                    byte = (w * NLD + i) * 256 + 4 * LANE[None, :]
                    voff = (byte // RB) * gs + byte % RB
                    g = np.arange(TK // 8, dtype=np.int64)
                    soff = (8 * g * gs)[:, None, None]
                    what = f"xg_gemm K={K} {kdim}x{ndim} nc={nc}"
                    _check_global(voff[None], soff, TK * gs, 0, TK * gs, what)
                    assert (nc * XG_TC * TB + voff[None] + soff).max() + 4 <= TK * gs, what
                    dst = (g[:, None, None] % XG_NG) * GB + (w * NLD + i[None]) * 256 + 4 * LANE[None, None, :]
                    _check_lds(dst, 0, XG_NG * GB, what)
            cap = min(MAX_GROUPED_PICKS, INT32_MAX // (kdim * 4))
            slots = np.array([0, cap - 1], dtype=np.int64)
            g = np.arange(TK // 8, dtype=np.int64)
            h = np.arange(XG_XROW // 256, dtype=np.int64)
            voff = (h[:, None] * 256 + 4 * LANE[None, :])
            soff = (slots[:, None] * kdim * 4 + g[None, :] * XG_XROW)[:, :, None, None]
            _check_global(voff[None, None], soff, cap * kdim * 4, 0, cap * kdim * 4, f"xg_gemm x K={K} {kdim}")
            for sl in (0, XG_MS - 1):
                for gg in range(XG_NG):
                    dst = XG_NG * GB + gg * XG_XGB + sl * XG_XROW + voff
                    _check_lds(dst, XG_NG * GB, lds, "xg_gemm x ring")


def test_model_reads_the_kernels_constants():
    """The constants the model uses are the kernels' (a change in a kernel changes the model with it)."""
    assert (NGRP, GU_NW, DN_NW) == (4, 4, 8)
    assert (GP_MT, GP_NW, GP_CPW, GP_NG, GP_XS) == (80, 8, 2, 2, 136)
    assert (XG_NW, XG_MS, XG_NG) == (8, 64, 2)
    assert MAX_DIM == 32768
    # at the largest registered shape a trellis matrix stays below 2^31 bytes
    assert MAX_DIM * MAX_DIM * 5 // 8 < 2 ** 31
