"""MI355X (gfx950) mixture-of-experts FFN layer of phoenix-lai's Gemma 4 26B-A4B path.

The compute lives in ``libphxmoe.so`` (hand-written HIP kernels behind the C ABI of
``include/phx_moe.h``); this package is the host-side binding used by the tests and the benchmark,
mirroring the three MoE call sites of the reference's ``GemmaGpu``:

* ``RecordMoe``      (src/GemmaGpu.cs:656-669): one token, shared-MLP output given
* ``RecordFfnMoe``   (src/GemmaGpu.cs:683-704): one token, dense shared FFN computed on the GPU
* ``RecordMoeRows``  (src/GemmaGpu.cs:850-882): T prompt rows

``gguf`` reads real models (GgufFile.Open and the MoE part of GemmaConfig.FromGguf).

There is no CPU fallback: loading fails loudly when the HIP library is missing.
"""
from .moe import (  # noqa: F401
    ArgumentError,
    GpuDeviceLostError,
    InvalidDataError,
    MoeContext,
    MoeError,
    NotSupportedError,
    OutOfDeviceMemoryError,
    LayerDesc,
    PHX,
    lib_path,
    load_lib,
)
from . import gguf, synth  # noqa: F401
