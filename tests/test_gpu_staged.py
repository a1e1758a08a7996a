"""Parity of the staged B=1 kernel on every shape it supports.

By default the library uses the staged kernel only for matrices of >= 28 MB
(it wins there); JUNO_STAGED_R forces it for all sizes (and sets the rows per
group).  Each check runs in one child process with the variables set, against
the CPU oracle, to the bar of the parity suite: max rel-err 1e-3 with
eps_r = 1e-3 * sum_c |w_rc x_c|.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r'''
import numpy as np
import oracle as O
from juno_amd import matvec as mv

be = mv.GpuContext.shared(0).create_mat_vec()
shapes = [
    (O.Q4_K, 5632, 2048), (O.Q4_K, 3001, 4096), (O.Q4_K, 1, 256), (O.Q4_K, 37, 768),
    (O.Q4_K, 700, 5632),            # 22 blocks: two column tiles
    (O.Q4_K, 300, 14336),           # 56 blocks: four column tiles
    (O.Q5_K, 3072, 3072), (O.Q5_K, 700, 5632), (O.Q5_K, 300, 14336), (O.Q5_K, 5, 256),
    (O.Q6_K, 2048, 5632), (O.Q6_K, 999, 3072), (O.Q6_K, 3, 256), (O.Q6_K, 513, 14336),
    (O.Q8_0, 2304, 3072), (O.Q8_0, 129, 8192), (O.Q8_0, 5, 32), (O.Q8_0, 77, 2080),
]
worst = 0.0
for qtype, rows, cols in shapes:
    rng = np.random.default_rng(rows * 7 + cols)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    if qtype == O.Q8_0:
        idx = rng.choice(w.size, max(w.size // 100, 1), replace=False)
        w[idx] *= 10
    x = rng.standard_normal(cols).astype(np.float32)
    x[::97] *= 50.0                 # a few large activations per block
    raw = O.quantize(qtype, w)
    deq = O.dequantize(qtype, raw, rows, cols).astype(np.float64)
    scale = np.abs(deq) @ np.abs(x.astype(np.float64))
    with be.upload_quant(qtype, rows, cols, raw) as dev:
        for a, b in [(0, rows), (rows // 3, rows - rows // 5)]:
            if b <= a:
                continue
            y = be.sgemv_quant(dev, x, a, b).astype(np.float64)
            ref = O.matvec(qtype, raw, x, a, b, cols).astype(np.float64)
            rel = np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3 * scale[a:b])
            worst = max(worst, float(rel.max()))
            print(qtype, rows, cols, a, b, f"{rel.max():.2e}", flush=True)
            assert rel.max() <= 1e-3, (qtype, rows, cols, a, b, rel.max())
# several matrices of one format sharing x in one staged launch (incl. column tiles)
import torch
for qtype, cols, rows_list in [(O.Q4_K, 4096, [333, 1000, 77]), (O.Q5_K, 3072, [700, 300]), (O.Q6_K, 14336, [129, 64]),
                               (O.Q8_0, 3072, [500, 501, 7, 90])]:
    rng = np.random.default_rng(cols + len(rows_list))
    x = rng.standard_normal(cols).astype(np.float32)
    dx = torch.from_numpy(x).cuda()
    mats, raws, dys = [], [], []
    for rows in rows_list:
        raw = O.quantize(qtype, (rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
        raws.append(raw)
        mats.append(be.upload_quant(qtype, rows, cols, raw))
        dys.append(torch.full((rows,), float("nan"), device="cuda"))
    be.sgemv_group_dev(mats, [dx.data_ptr()] * len(mats), [d.data_ptr() for d in dys])
    torch.cuda.synchronize()
    for rows, raw, dy, m in zip(rows_list, raws, dys, mats):
        y = dy.cpu().numpy().astype(np.float64)
        ref = O.matvec(qtype, raw, x, 0, rows, cols).astype(np.float64)
        deq = O.dequantize(qtype, raw, rows, cols).astype(np.float64)
        rel = np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3 * (np.abs(deq) @ np.abs(x.astype(np.float64))))
        print("group", qtype, rows, cols, f"{rel.max():.2e}", flush=True)
        assert rel.max() <= 1e-3, (qtype, rows, cols, rel.max())
        m.close()
# no column-tile ring wait gave up (jh_sync_faults counts them)
import ctypes
from juno_amd import _lib
nf = ctypes.c_uint(7)
assert _lib.load().jh_sync_faults(0, ctypes.byref(nf)) == 0 and nf.value == 0, nf.value
print("staged-ok", worst)
'''


@pytest.mark.parametrize("rows_per_group,wide", [("2", None), ("1", None), ("2", "4")],
                         ids=["two rows", "one row (wide default)", "per-lane x for column tiles"])
def test_staged_kernel_all_shapes(rows_per_group, wide):
    """Every shape through the staged kernel with two rows per group, with one
    (the default for column-tiled rows: 16 waves sharing one LDS image of x), and
    with column-tiled rows converting x per lane (JUNO_STAGED_WIDE=4)."""
    env = dict(os.environ, JUNO_STAGED_R=rows_per_group)
    if wide:
        env["JUNO_STAGED_WIDE"] = wide
    r = subprocess.run([sys.executable, "-u", "-c", CHILD], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0 and "staged-ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
