"""juno_amd -- MI355X-native (gfx950) quantized matvec hot path of Juno.

The compute lives in ``libjunohip.so`` (hand-written HIP kernels behind the C ABI
of ``include/junohip.h``); this package is the host-side mirror of the
reference's matvec interface (``juno_amd.matvec``).
"""
from .matvec import (F32, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, DeviceQuantMatrix, GpuContext, HipMatVec,  # noqa: F401
                     IllegalArgumentException, IllegalStateException, IOException, MatVecBackend, QuantizedTensor,
                     UnsupportedOperationException, device_count, device_info, raw_byte_count)

from .gguf import GgufArray, GgufReader  # noqa: F401,E402

__version__ = "0.1.0"
