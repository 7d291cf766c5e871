"""LDS bank model of the one-pass 2D kernel (fft2d_small_body,
ferrum-gpu_amd/csrc/kernels/fft_2d_small.hpp): the per-shape layouts of
small2d_layout must not conflict more than the first layout (pitch
C + C/16 + 1, exchanges padded one slot per 16, consecutive lanes per line).

Model: 32 four-byte banks; a 64-bit access serves 16 lanes per cycle, and a
cycle costs as many passes as the most distinct dwords any bank receives.
The model reproduces the conflict rates rocprof measured on the first layout
(SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT): 16x16
0.37, 32x32 0.75, 64x64 0.72, 128x128 0.61 against 0.40 / 0.70 / 0.70 / 0.60
modelled).  Plain phases (load, store, row and column reads and writes) use
the layout's pitch; exchanges follow the Stockham destinations of
tests/test_stockham_model.py.
"""

from __future__ import annotations

import numpy as np
import pytest

from test_fft2d_small_model import lanes, layout, shapes


def loge(lr, lc):
    """Elements per thread of the LDS-resident kernel (fft2d_small_body): 8, 16
    for 16384 points.  The rates below were measured on it for shapes that now
    run the register-resident kernel (64x64, 128x128), so the model keeps its
    geometry rather than today's dispatch."""
    return 4 if lr + lc >= 14 else 3


def fpi(lr, lc):
    """Images per workgroup of the LDS-resident kernel (256 threads, or one image)."""
    t = (1 << (lr + lc)) >> loge(lr, lc)
    return 1 if t >= 256 else 256 // t


def cycles(addr):
    a = np.asarray(addr)
    tot = 0
    for g in range(0, 64, 16):
        dw = np.unique(np.concatenate([2 * a[g:g + 16], 2 * a[g:g + 16] + 1]))
        tot += np.bincount(dw % 32, minlength=32).max()
    return tot / 4.0


def dst(log_n, log_e, s, t, i, q):
    n, e = 1 << log_n, 1 << log_e
    logr = log_e if s < log_n // log_e else log_n % log_e
    L = 1 << (s * log_e)
    b = t + (n // e) * i
    return (b >> (s * log_e)) * L * (1 << logr) + (b & (L - 1)) + q * L


def exchanges(log_n, log_e, t, sh):
    """Per exchange instruction: each lane's padded position (scatters, then gathers)."""
    n, e = 1 << log_n, 1 << log_e
    nstages = log_n // log_e + (1 if log_n % log_e else 0)
    out = []
    for s in range(nstages - 1):
        logr = log_e if s < log_n // log_e else log_n % log_e
        for i in range(e >> logr):
            for q in range(1 << logr):
                p = dst(log_n, log_e, s, t, i, q)
                out.append(p + (p >> sh))
        for m in range(e):
            p = t + (n // e) * m
            out.append(p + (p >> sh))
    return out


def conflict_rate(lr, lc, lay):
    R, C = 1 << lr, 1 << lc
    le = loge(lr, lc)
    E = 1 << le
    TC, TR, TIMG = C // E, R // E, (R * C) >> le
    block = fpi(lr, lc) * TIMG
    P, CP, img = lay["P"], lay["CP"], R * lay["P"]
    rr, rt = lanes(TIMG, TC, lay["row_tm"])
    cc, ct = lanes(TIMG, TR, lay["col_tm"])
    spent = ideal = 0.0
    for w in range(block // 64):
        tid = np.arange(64 * w, 64 * w + 64)
        slot, local = tid // TIMG, tid % TIMG
        acc = []
        for j in range(E):
            e = tid + block * j
            n = e & (R * C - 1)
            acc.append((e >> (lr + lc)) * img + (n >> lc) * P + (n & (C - 1)))
        r, t = rr[local], rt[local]
        acc += [slot * img + r * P + t + TC * m for m in range(E)]
        acc += [slot * img + r * P + x for x in exchanges(lc, le, t, lay["shr"])]
        c, t = cc[local], ct[local]
        acc += [slot * img + (t + TR * m) * P + c for m in range(E)]
        acc += [slot * img + c * CP + x for x in exchanges(lr, le, t, lay["shc"])]
        spent += sum(cycles(a) for a in acc)
        ideal += len(acc)
    return spent / ideal - 1.0


def first_layout(lr, lc):
    R, C = 1 << lr, 1 << lc
    return dict(P=C + C // 16 + 1, CP=R + R // 16, shr=4, shc=4, row_tm=False, col_tm=False)


def test_model_reproduces_the_measured_rates():
    measured = {(4, 4): 0.373, (5, 5): 0.747, (6, 6): 0.722, (7, 7): 0.611}
    for (lr, lc), rate in measured.items():
        assert abs(conflict_rate(lr, lc, first_layout(lr, lc)) - rate) < 0.06


@pytest.mark.parametrize("lr,lc", shapes())
def test_layout_conflicts_no_more_than_the_first(lr, lc):
    new, old = conflict_rate(lr, lc, layout(lr, lc)), conflict_rate(lr, lc, first_layout(lr, lc))
    assert new <= old + 1e-9
    assert new <= 0.3
    # the same occupancy: no fewer workgroups per CU by LDS
    R, C = 1 << lr, 1 << lc
    lds_new, lds_old = fpi(lr, lc) * R * layout(lr, lc)["P"] * 8, fpi(lr, lc) * R * first_layout(lr, lc)["P"] * 8
    assert 163840 // lds_new >= 163840 // lds_old
