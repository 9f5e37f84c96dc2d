"""MI355X-native (gfx950) MXFP4 mixture-of-experts path of GPT-OSS, behind a C ABI that
replaces the GPU backend of gabearro/SilentOTITHRanDouSha (src/gpu/moe_dispatch.rs).

The compute lives in libmxfp4moe.so (HIP kernels, built by __graft_entry__.build()); this
package is a thin host front end. Importing it does not need a GPU; creating a dispatcher
does, and fails loudly without the library or a gfx950 device.
"""
from ._ffi import LIB_PATH, MoeError, lib  # noqa: F401
from .dispatcher import (DeviceBuffer, GpuMoeDispatcher, mxfp4_dequant, mxfp4_matvec,  # noqa: F401
                         mxfp4_pack, safetensors_find)
from .beaver import GpuTripleGen32  # noqa: F401

(KERNEL_ROUTE, KERNEL_BUCKET, KERNEL_GATE_UP, KERNEL_DOWN, KERNEL_COMBINE, KERNEL_DECODE_GATE_UP,
 KERNEL_DECODE_DOWN, KERNEL_DECODE_LAYER, KERNEL_RESERVED, KERNEL_NORM) = range(10)
