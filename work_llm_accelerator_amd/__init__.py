"""MI355X-native (gfx950) implementation of the quantized Qwen2.5-1.5B decoder-layer hot path.

The product is the HIP library under _lib/ (built by work_llm_accelerator_amd.build): the
reference's decode/prefill C ABI as a drop-in, plus a device-resident multi-layer API.  The
Python modules here are the host side above that C ABI: ctypes bindings (abi), the DDR layout
and descriptors (layout), the INT4 quantizer and bf16 rounding (quant).
"""

from . import layout, quant  # noqa: F401

__all__ = ["layout", "quant"]
