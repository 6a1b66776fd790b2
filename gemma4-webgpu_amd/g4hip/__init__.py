"""Python host for libg4hip.so, the MI355X decode hot path of gemma4-webgpu.

This package is a thin ctypes layer over the C ABI in ``include/g4hip.h``.
It owns no compute: every kernel runs in the HIP library, and importing this
package fails loudly when the library has not been built (there is no CPU
fallback). Kernel wrappers keep the reference's kernel keys
(src/shaders.ts:34-56) and Params field order.
"""
from __future__ import annotations

from ._lib import (  # noqa: F401
    G4Error,
    LIB_PATH,
    O_SHARES,
    lib,
    MatmulParams,
    KvStoreParams,
    AttnScoreParams,
    SoftmaxParams,
    AttnOutputParams,
    AttnFusedParams,
    PagedAttnParams,
    PerHeadNormParams,
    NormRopeParams,
    RmsNormParams,
    NormAddParams,
    SoftcapParams,
)
from .device import Context, Buffer  # noqa: F401
