"""neso_amd: MI355X-native (gfx950) kernels for neso's hot path.

Flash-Attention-2 forward, relative-position-bias FA2 and weight-only
quantised matmuls, hand-written in HIP and exposed through the C ABI in
``include/neso_amd.h``.  The Python layer only validates, picks the HIP
stream and calls the library; there is no CPU implementation.
"""
from ._lib import (  # noqa: F401
    NESO_BIAS_DENSE_SCALED_F16,
    NESO_BIAS_TABLE_F32,
    NESO_EINVAL,
    NESO_ELAUNCH,
    NESO_EUNSUPPORTED,
    NESO_IO_F16,
    NESO_IO_F32,
    NESO_OK,
    NESO_OUT_F16,
    NESO_OUT_F32,
    NesoArgumentError,
    NesoError,
)
from .kernels import (  # noqa: F401
    KERNELS,
    attention,
    flash_attention_fwd,
    flash_attention_io_fwd,
    flash_attention_window_fwd,
    launch,
    launch_plan,
    manifest,
    precompute_bias_and_qu,
    rel_pos_attention,
    rel_pos_fa2_fwd,
    rel_pos_precompute,
    w4a16_linear,
    w4a16_matmul,
    w8a16_matmul,
    w8a16_scaled_matmul,
    window_attention,
)
from .packing import pack_int4, unpack_int4  # noqa: F401

__version__ = "0.1.0"
