"""juno.MatVec ranges under rocprofv3: a few resident matVecs of TinyLlama
shapes through the HipMatVec backend, for

    JUNO_ROCTX=1 rocprofv3 --marker-trace --kernel-trace --stats -d out -o demo -- python3 -m juno_amd.trace_demo

Each call pushes a roctx range "juno.MatVec backend=<label> rows=R cols=C
batch=B" (the reference's JFR event, MatVecEvent.java:46-72), which the
marker trace lists next to the kernels the call launched.
"""
from __future__ import annotations

import numpy as np


def main() -> None:
    import torch

    from juno_amd import matvec as mv

    be = mv.GpuContext.shared(0).create_mat_vec()
    x = np.random.default_rng(0).standard_normal(2048).astype(np.float32)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    for qtype, rows in ((mv.Q4_K, 5632), (mv.Q6_K, 256), (mv.Q8_0, 2048)):
        w = torch.randn(rows * 2048, generator=g, device="cuda").mul_(0.02)
        dev = be.quantize_dev(qtype, w.data_ptr(), rows, 2048, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        with dev:
            for _ in range(3):
                be.sgemv_quant(dev, x)
            be.sgemv_batched(dev, np.tile(x, (16, 1)))
    print("trace demo done", flush=True)


if __name__ == "__main__":
    main()
