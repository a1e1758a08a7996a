"""Per-wave timeline of the staged B = 1 walk (the dominant kernel: the grouped
Q4_K [ffn_gate, ffn_up] launch at Llama-3-8B shapes, 2 x 14336 x 4096).

Two steps, because the instrumented library is built on the CPU and run on the
GPU box:

    python -m juno_amd.timeline build    # juno_amd/_timeline/libjunohip.so, compiled with -DJH_TIMELINE
    python -m juno_amd.timeline run      # the launches and the summary (markdown on stdout)
    python -m juno_amd.timeline down     # the same for the Q6_K ffn_down (column-tiled rows)
    python -m juno_amd.timeline mfma 32  # the batched MFMA walk at B <= 32 (per super-block step)

The instrumented build stamps s_memrealtime (100 MHz) per wave of the DYN walk
at entry, after the x prologue's barrier, once its first row group has landed
in LDS, and at the end of its walk (jh_debug_timeline).  The shipped library
has no stamps (jh_debug_timeline returns JH_EUNSUPPORTED there).  Each launch
is timed relative to its earliest wave start; the summary gives medians and
spreads over launches, with the weights of 8 distinct layers so that no launch
finds its matrices in the 256 MB MALL.  The MFMA variant stamps each wave of
the B <= 32 walk at entry and, per super-block step, after the step's barrier,
once its weight chunks are parked in LDS, once the next x is staged and after
its MFMAs and fold (jh_debug_timeline kernel 1).
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_timeline")
LIB = os.path.join(OUT_DIR, "libjunohip.so")
FLAGS = "-DJH_TIMELINE"
HIDDEN, FFN, LAYERS, REPS = 4096, 14336, 8, 4
TICK_NS = 10.0  # s_memrealtime runs at 100 MHz


def build() -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    env = dict(os.environ, JH_EXTRA_FLAGS=FLAGS, JUNO_LIB_OUT=LIB)
    subprocess.run([sys.executable, "-m", "juno_amd.build"], env=env, check=True, cwd=os.path.dirname(HERE))
    return LIB


def _pct(a, q):
    import numpy as np
    return float(np.percentile(a, q))


def staged_launch_stats(raw, waves_per_wg: int = 16) -> dict:
    """One launch's staged-walk stamps (4 per wave: entry, prologue barrier,
    first row group landed, walk end; 0 for waves that did not run), in µs
    from the launch's earliest wave start."""
    import numpy as np
    t = np.asarray(raw, dtype=np.uint64).reshape(-1, 4).astype(np.int64)
    t = t[t[:, 0] > 0]
    base = t[:, 0].min()
    rel = (t - base) * TICK_NS / 1e3
    wg_end = rel[:, 3].reshape(-1, waves_per_wg).max(axis=1)
    return {
        "waves": int(len(rel)),
        "start_p50": _pct(rel[:, 0], 50), "start_p90": _pct(rel[:, 0], 90), "start_max": float(rel[:, 0].max()),
        "prologue_p50": _pct(rel[:, 1], 50), "prologue_p90": _pct(rel[:, 1], 90),
        "first_rows_p10": _pct(rel[:, 2], 10), "first_rows_p50": _pct(rel[:, 2], 50),
        "first_rows_p90": _pct(rel[:, 2], 90),
        "wg_end_min": float(wg_end.min()), "wg_end_p10": _pct(wg_end, 10), "wg_end_p50": _pct(wg_end, 50),
        "wg_end_p90": _pct(wg_end, 90), "end": float(rel[:, 3].max()),
    }


MFMA_PER_WAVE = 68  # entry, 4 per super-block step (up to 16), 3 in the split-K epilogue


def mfma_launch_stats(raw) -> dict:
    """One launch's batched-walk stamps (MFMA_PER_WAVE per wave), in µs from the
    launch's earliest wave start: per step, the wait at its barrier (from the
    previous step's fold, or from entry for the first), the park, the staging
    of the next x and the MFMAs and fold; then the epilogue."""
    import numpy as np
    t = np.asarray(raw, dtype=np.uint64).reshape(-1, MFMA_PER_WAVE).astype(np.int64)
    t = t[t[:, 0] > 0]
    steps = int(((t[:, 1:65] > 0).sum(axis=1) // 4).min())
    base = t[:, 0].min()
    epi = (t[:, 65:68] - base) * TICK_NS / 1e3  # partials acknowledged, arrival counted, end (last split)
    rel = (t[:, : 1 + 4 * steps] - base) * TICK_NS / 1e3
    st = rel[:, 1:].reshape(len(rel), steps, 4)
    prev = np.concatenate([rel[:, :1], st[:, :-1, 3]], axis=1)  # end of the previous step
    parts = {"barrier": st[:, :, 0] - prev, "park": st[:, :, 1] - st[:, :, 0],
             "stage_issue": st[:, :, 2] - st[:, :, 1], "mfma_fold": st[:, :, 3] - st[:, :, 2]}
    d = {"waves": int(len(rel)), "steps": steps,
         "start_p50": _pct(rel[:, 0], 50), "start_max": float(rel[:, 0].max()),
         "first_step_p50": _pct(st[:, 0, 0], 50), "walk_end_p50": _pct(st[:, -1, 3], 50),
         "walk_end_max": float(st[:, -1, 3].max())}
    acked = t[:, 65] > 0  # waves that went through the split-K hand-off
    if acked.any():
        d["acked_p50"] = _pct(epi[acked, 0] - st[acked, -1, 3], 50)
        d["acked_p90"] = _pct(epi[acked, 0] - st[acked, -1, 3], 90)
        d["counted_p50"] = _pct(epi[acked, 1] - epi[acked, 0], 50)
        d["counted_p90"] = _pct(epi[acked, 1] - epi[acked, 0], 90)
    last = t[:, 67] > 0  # waves of the splits that summed the partials
    if last.any():
        d["sum_store_p50"] = _pct(epi[last, 2] - epi[last, 1], 50)
        d["end_max"] = float(epi[last, 2].max())
    for k, v in parts.items():
        d[k + "_first"] = _pct(v[:, 0], 50)
        d[k + "_rest"] = _pct(v[:, 1:], 50) if steps > 1 else 0.0
        d[k + "_rest_p90"] = _pct(v[:, 1:], 90) if steps > 1 else 0.0
    return d


def run_child(kind: str = "gate_up") -> dict:
    """kind gate_up: the grouped Q4_K [gate, up] launch; down: the Q6_K ffn_down
    (4096 x 14336, column-tiled rows)."""
    import ctypes

    import numpy as np
    import torch

    from juno_amd import _lib
    from juno_amd import matvec as mv

    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    s = torch.cuda.current_stream()
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    down = kind == "down"
    n, qt, rows, cols = (1, mv.Q6_K, HIDDEN, FFN) if down else (2, mv.Q4_K, FFN, HIDDEN)
    mats = []
    for _ in range(LAYERS):
        pair = []
        for _ in range(n):
            w = torch.randn(rows * cols, generator=g, device="cuda").mul_(0.02)
            pair.append(be.quantize_dev(qt, w.data_ptr(), rows, cols, s.cuda_stream))
            del w
        mats.append(pair)
    torch.cuda.synchronize()
    x = torch.randn(cols, generator=g, device="cuda")
    ys = [torch.empty(rows, device="cuda") for _ in range(n)]
    V = ctypes.c_void_p
    n_slots = 4096 * 4
    buf = (ctypes.c_uint64 * n_slots)()
    launches = []
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for rep in range(REPS + 1):
        for pair in mats:
            hs = (V * n)(*[m.handle for m in pair])
            xs = (V * n)(*[x.data_ptr()] * n)
            yp = (V * n)(*[y.data_ptr() for y in ys])
            ctypes.memset(buf, 0, ctypes.sizeof(buf))
            e0.record(s)
            if L.jh_qmatvec_group_dev(n, hs, xs, yp, V(s.cuda_stream)):
                raise RuntimeError(_lib.last_error())
            e1.record(s)
            torch.cuda.synchronize()
            if L.jh_debug_timeline(0, 0, buf, n_slots):
                raise RuntimeError(_lib.last_error())
            if rep == 0:
                continue  # warm-up pass
            d = staged_launch_stats(np.frombuffer(buf, dtype=np.uint64))
            d["event_us"] = float(e0.elapsed_time(e1) * 1e3)
            launches.append(d)
    for pair in mats:
        for m in pair:
            m.close()
    return {"launches": launches, "kind": kind,
            "bytes": n * rows * (cols // 256) * (210 if down else 144) + 4 * (cols + n * rows)}


def run_child_mfma(B: int = 32) -> dict:
    """The grouped [gate, up] MFMA launch at batch B: per wave and super-block
    step, time waiting at the step's barrier, parking the weight chunks (waits
    on their global loads), staging the next x (and issuing the next loads), and
    the MFMAs plus the fold."""
    import ctypes

    import numpy as np
    import torch

    from juno_amd import _lib
    from juno_amd import matvec as mv

    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    s = torch.cuda.current_stream()
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    mats = []
    for _ in range(LAYERS):
        pair = []
        for _ in range(2):
            w = torch.randn(FFN * HIDDEN, generator=g, device="cuda").mul_(0.02)
            pair.append(be.quantize_dev(mv.Q4_K, w.data_ptr(), FFN, HIDDEN, s.cuda_stream))
            del w
        mats.append(pair)
    torch.cuda.synchronize()
    X = torch.randn(B, HIDDEN, generator=g, device="cuda")
    ys = [torch.empty(B, FFN, device="cuda") for _ in range(2)]
    V = ctypes.c_void_p
    kernel, ksplit = ctypes.c_int(), ctypes.c_int()
    hs0 = (V * 2)(mats[0][0].handle, mats[0][1].handle)
    if L.jh_qmatvec_batched_plan(2, hs0, B, ctypes.byref(kernel), ctypes.byref(ksplit)):
        raise RuntimeError(_lib.last_error())
    n_slots = 512 * 8 * MFMA_PER_WAVE
    buf = (ctypes.c_uint64 * n_slots)()
    launches = []
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for rep in range(REPS + 1):
        for pair in mats:
            hs = (V * 2)(pair[0].handle, pair[1].handle)
            xs = (V * 2)(X.data_ptr(), X.data_ptr())
            yp = (V * 2)(ys[0].data_ptr(), ys[1].data_ptr())
            ctypes.memset(buf, 0, ctypes.sizeof(buf))
            e0.record(s)
            if L.jh_qmatvec_batched_group_dev(2, hs, xs, B, yp, V(s.cuda_stream)):
                raise RuntimeError(_lib.last_error())
            e1.record(s)
            torch.cuda.synchronize()
            if L.jh_debug_timeline(0, 1, buf, n_slots):
                raise RuntimeError(_lib.last_error())
            if rep == 0:
                continue
            d = mfma_launch_stats(np.frombuffer(buf, dtype=np.uint64))
            d["event_us"] = float(e0.elapsed_time(e1) * 1e3)
            launches.append(d)
    for pair in mats:
        for m in pair:
            m.close()
    return {"launches": launches, "B": B, "kernel": kernel.value, "ksplit": ksplit.value}


def summary_mfma(res: dict) -> str:
    import numpy as np
    ls = res["launches"]

    def med(k):
        return float(np.median([d.get(k, float("nan")) for d in ls]))
    out = [f"B = {res['B']}, plan kernel {res['kernel']} K split {res['ksplit']}, {ls[0]['waves']} waves, "
           f"{ls[0]['steps']} super-block steps per wave; medians over {len(ls)} launches.", "",
           "| quantity (µs) | value |", "|---|---:|",
           f"| HIP-event duration of the eager launch | {med('event_us'):.2f} |",
           f"| waves started: median / last | {med('start_p50'):.2f} / {med('start_max'):.2f} |",
           f"| first step's barrier passed (median wave) | {med('first_step_p50'):.2f} |",
           f"| walk end: median wave / last wave | {med('walk_end_p50'):.2f} / {med('walk_end_max'):.2f} |",
           f"| epilogue: partials acknowledged after the walk, median (p90) | {med('acked_p50'):.2f} ({med('acked_p90'):.2f}) |",
           f"| epilogue: arrival counted after that, median (p90) | {med('counted_p50'):.2f} ({med('counted_p90'):.2f}) |",
           f"| epilogue (last split): partial sums and stores, median | {med('sum_store_p50'):.2f} |",
           f"| last wave done | {med('end_max'):.2f} |",
           "", "| per step, median wave (p90) | first step | later steps |", "|---|---:|---:|"]
    for k in ("barrier", "park", "stage_issue", "mfma_fold"):
        out.append(f"| {k} | {med(k + '_first'):.2f} | {med(k + '_rest'):.2f} ({med(k + '_rest_p90'):.2f}) |")
    return "\n".join(out)


def summary(res: dict) -> str:
    import numpy as np
    ls = res["launches"]
    bytes_launch = res.get("bytes", 2 * FFN * (HIDDEN // 256) * 144 + 4 * (HIDDEN + 2 * FFN))

    def med(k):
        return float(np.median([d[k] for d in ls]))
    walk = med("wg_end_p50") - med("first_rows_p50")
    rows = [
        ("HIP-event duration of the eager launch", med("event_us")),
        ("waves started: median / p90 / last", f"{med('start_p50'):.2f} / {med('start_p90'):.2f} / {med('start_max'):.2f}"),
        ("x prologue done (barrier): median / p90", f"{med('prologue_p50'):.2f} / {med('prologue_p90'):.2f}"),
        ("first row group landed: p10 / median / p90",
         f"{med('first_rows_p10'):.2f} / {med('first_rows_p50'):.2f} / {med('first_rows_p90'):.2f}"),
        ("workgroup walk end: first / p10 / median / p90",
         f"{med('wg_end_min'):.2f} / {med('wg_end_p10'):.2f} / {med('wg_end_p50'):.2f} / {med('wg_end_p90'):.2f}"),
        ("last wave done", med("end")),
        ("steady-state rate: bytes / (median end - median first rows), TB/s", bytes_launch / (walk * 1e-6) / 1e12),
    ]
    out = ["| quantity (µs from the launch's first wave start) | value |", "|---|---:|"]
    for k, v in rows:
        out.append(f"| {k} | {v if isinstance(v, str) else f'{v:.2f}'} |")
    out.append("")
    out.append(f"{len(ls)} launches ({LAYERS} layers' distinct weights x {REPS}), "
               f"{ls[0]['waves']} waves each; medians over launches.")
    return "\n".join(out)


def main(argv) -> None:
    cmd = argv[1] if len(argv) > 1 else "run"
    if cmd == "build":
        print(build())
        return
    if cmd == "child":
        print(json.dumps(run_child(argv[2] if len(argv) > 2 else "gate_up")))
        return
    if cmd == "child_mfma":
        print(json.dumps(run_child_mfma(int(argv[2]) if len(argv) > 2 else 32)))
        return
    if not os.path.exists(LIB):
        raise SystemExit(f"{LIB} is not built: run `python -m juno_amd.timeline build` first")
    env = dict(os.environ, JUNO_LIB_PATH=LIB, JH_EXTRA_FLAGS=FLAGS)
    mfma = cmd == "mfma"
    child = ["child_mfma", argv[2] if len(argv) > 2 else "32"] if mfma else ["child", "down" if cmd == "down" else "gate_up"]
    r = subprocess.run([sys.executable, "-m", "juno_amd.timeline", *child], env=env, capture_output=True, text=True,
                       cwd=os.path.dirname(HERE))
    if r.returncode:
        raise SystemExit(r.stderr[-4000:])
    res = json.loads(r.stdout.strip().splitlines()[-1])
    print(summary_mfma(res) if mfma else summary(res))
    # run [json], down [json], mfma [B [json]]
    out = (argv[3] if len(argv) > 3 else None) if mfma else (argv[2] if len(argv) > 2 else None)
    if out:
        with open(out, "w") as f:
            json.dump(res, f, indent=1)


if __name__ == "__main__":
    main(sys.argv)
