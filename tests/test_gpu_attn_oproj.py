"""Attention and the output projection in one call
(jh_rope_attention_qmatvec_dev): rope, KV append and gqa, then y = wo . att
(transformerLayer, LlamaTransformerHandler.java:765-776).  By default the pair
of launches; with JUNO_ATTN_FUSE=1, where the staged GEMV applies, attention's
combine of its chunk partials runs in the GEMV's input conversion instead of
its own launch.

Checked against jh_rope_attention_dev on copies of the same cache (the pair's
first half), by default and in a child process with JUNO_ATTN_FUSE=1:
  * att bit for bit (the prologue repeats attn_combine_k's arithmetic in its
    order), and the caches alike;
  * y against the oracle's quantized matvec of that att: the GEMV bar, per-row
    |err| / max(|ref|, 1e-3 sum_c |w_rc att_c|) <= 1e-3;
  * in a child process with JUNO_ATTN_FUSE=1 and JUNO_STAGED_R=1 (the plain call
    then takes the same staged walk): y bit for bit equal to jh_qmatvec_dev on
    att, also for an att whose outliers send the walk to its exact path.
Shapes: Llama-3-8B (32 / 8 heads of 128, wo 4096 x 4096) and TinyLlama (32 / 4
of 64, 2048 x 2048) with Q4_K / Q6_K / Q8_0 wo; 16 and 64 chunks (fused), and
a cache of 8192 positions (128 chunks: the pair of launches).
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from juno_amd import _lib  # noqa: E402
from juno_amd import matvec as mv  # noqa: E402

V = ctypes.c_void_p
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def say(*a):
    print(*a, flush=True)


def P(t):
    return V(t.data_ptr())


def wo_matrix(be, qt, rows, cols, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.randn(rows * cols, generator=g, device="cuda").mul_(0.02)
    m = be.quantize_dev(qt, w.data_ptr(), rows, cols, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return m


def run_case(L, m, nh, nkv, hd, max_seq, pos, seed, outlier=False):
    """The fused call and jh_rope_attention_dev on copies of one cache: (att, y, att_pair)."""
    kvd = nkv * hd
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal(n).astype(np.float32) for n in (nh * hd, kvd, kvd))
    kc = torch.randn(max_seq, kvd, device="cuda", generator=torch.Generator(device="cuda").manual_seed(seed))
    vc = torch.randn(max_seq, kvd, device="cuda", generator=torch.Generator(device="cuda").manual_seed(seed + 1))
    if outlier:  # one dimension of each KV head 1e6, the rest ~1e-4: att has groups with one outlier
        vc.mul_(1e-4)
        vc.view(max_seq, nkv, hd)[:, :, 0] = 1e6
        v = (v * 1e-4).astype(np.float32)
        v.reshape(nkv, hd)[:, 0] = 1e6
    kc2, vc2 = kc.clone(), vc.clone()
    dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, k, v))
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    att = torch.full((nh * hd,), float("nan"), device="cuda")
    att2 = torch.full((nh * hd,), float("nan"), device="cuda")
    y = torch.full((m.rows,), float("nan"), device="cuda")
    rc = L.jh_rope_attention_qmatvec_dev(P(dq), P(dk), P(dv), nh, nkv, hd, P(dpos), max_seq, ctypes.c_float(10000.0),
                                         P(kc), P(vc), m.handle, P(att), P(y), None)
    assert rc == 0, _lib.last_error()
    rc = L.jh_rope_attention_dev(P(dq), P(dk), P(dv), nh, nkv, hd, P(dpos), max_seq, ctypes.c_float(10000.0),
                                 P(kc2), P(vc2), P(att2), None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    return att.cpu().numpy(), y.cpu().numpy(), att2.cpu().numpy()


CASES = [
    (32, 8, 128, O.Q4_K, 512, 511),    # Llama-3-8B, 16 chunks of 32
    (32, 8, 128, O.Q4_K, 512, 0),      # one position: one chunk
    (32, 8, 128, O.Q6_K, 512, 100),
    (32, 8, 128, O.Q8_0, 512, 257),
    (32, 8, 128, O.Q4_K, 2048, 1999),  # 64 chunks: the most the prologue takes
    (32, 8, 128, O.Q4_K, 8192, 700),   # 128 chunks: attention's own combine, then the GEMV
    (32, 4, 64, O.Q4_K, 512, 300),     # TinyLlama
]


@pytest.mark.parametrize("nh,nkv,hd,qt,max_seq,pos", CASES)
def test_attention_output_projection(nh, nkv, hd, qt, max_seq, pos):
    check_case(nh, nkv, hd, qt, max_seq, pos)


def check_case(nh, nkv, hd, qt, max_seq, pos):
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    cols = nh * hd
    m = wo_matrix(be, qt, cols, cols, 2100 + pos)
    try:
        say(f"attention + wo: heads {nh}/{nkv} x {hd}, type {qt}, max_seq {max_seq}, pos {pos}")
        att, y, att2 = run_case(L, m, nh, nkv, hd, max_seq, pos, 2200 + pos)
        assert np.array_equal(att, att2), np.abs(att - att2).max()
        raw = m.packed_bytes()
        absdeq = np.abs(O.dequantize(qt, raw, cols, cols).astype(np.float64))
        ref = O.matvec(qt, raw, att2, 0, cols, cols, nthreads=16).astype(np.float64)
        scale = absdeq @ np.abs(att2.astype(np.float64))
        err = np.abs(y.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3 * scale)
        say(f"  y vs oracle: max rel-err {err.max():.2e}")
        assert err.max() <= 1e-3
    finally:
        m.close()


def test_attention_output_projection_arguments():
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    m = wo_matrix(be, O.Q4_K, 512, 1024, 2300)
    try:
        d = torch.zeros(4096, device="cuda")
        pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        # wo has 1024 columns, attention gives 8 x 64 = 512
        rc = L.jh_rope_attention_qmatvec_dev(P(d), P(d), P(d), 8, 8, 64, P(pos), 4, ctypes.c_float(1e4), P(d), P(d),
                                             m.handle, P(d), P(d), None)
        assert rc == _lib.JH_EINVAL and "columns" in _lib.last_error()
        rc = L.jh_rope_attention_qmatvec_dev(P(d), P(d), P(d), 16, 8, 64, P(pos), 4, ctypes.c_float(1e4), P(d), P(d),
                                             m.handle, None, P(d), None)
        assert rc == _lib.JH_EINVAL
        # att and y overlap
        y = torch.zeros(4096, device="cuda")
        rc = L.jh_rope_attention_qmatvec_dev(P(d), P(d), P(d), 16, 8, 64, P(pos), 4, ctypes.c_float(1e4), P(d), P(d),
                                             m.handle, P(y), V(y.data_ptr() + 4 * 100), None)
        assert rc == _lib.JH_EINVAL and "overlap" in _lib.last_error()
    finally:
        m.close()


FUSED_CHILD = r"""
import sys
sys.path.insert(0, "tests")
from test_gpu_attn_oproj import CASES, check_case
for c in CASES:
    check_case(*c)
print("fused-ok", flush=True)
"""


def test_attention_output_projection_fused():
    env = dict(os.environ, JUNO_ATTN_FUSE="1")
    r = subprocess.run([sys.executable, "-u", "-c", FUSED_CHILD], env=env, cwd=ROOT, capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0 and "fused-ok" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]


CHILD = r"""
import ctypes, sys
import numpy as np, torch
sys.path.insert(0, "tests")
import oracle as O
from juno_amd import _lib
from juno_amd import matvec as mv
from test_gpu_attn_oproj import P, run_case, wo_matrix
L = _lib.load()
be = mv.GpuContext.shared(0).create_mat_vec()
for nh, nkv, hd, qt, pos, outlier in ((32, 8, 128, O.Q4_K, 511, False), (32, 8, 128, O.Q4_K, 40, True),
                                      (32, 4, 64, O.Q6_K, 200, False)):
    cols = nh * hd
    m = wo_matrix(be, qt, cols, cols, 2400 + pos)
    print("staged comparison", nh, nkv, hd, qt, pos, outlier, flush=True)
    att, y, att2 = run_case(L, m, nh, nkv, hd, 512, pos, 2500 + pos, outlier)
    assert np.array_equal(att, att2)
    da = torch.from_numpy(att2).cuda()
    y2 = torch.full((cols,), float("nan"), device="cuda")
    assert L.jh_qmatvec_dev(m.handle, P(da), P(y2), 0, cols, None) == 0, _lib.last_error()
    torch.cuda.synchronize()
    y2 = y2.cpu().numpy()
    assert np.isfinite(y).all()
    assert np.array_equal(y, y2), np.abs(y - y2).max()
    m.close()
print("comb-ok", flush=True)
"""


def test_attention_output_projection_matches_staged_walk():
    env = dict(os.environ, JUNO_STAGED_R="1", JUNO_ATTN_FUSE="1")
    r = subprocess.run([sys.executable, "-u", "-c", CHILD], env=env, cwd=ROOT, capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0 and "comb-ok" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]
