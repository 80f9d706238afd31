"""flyai_amd: MI355X (gfx950) stage-step library for a GPT-OSS-shaped MXFP4 MoE pipeline stage.

The compute lives in libflyai_stage.so (hand-written HIP kernels behind the C ABI declared in
include/flyai_stage.h); this package is the Python host side: ctypes bindings (_lib), torch tensor
wrappers (ops), weights, rotary tables, and the stage runtimes (runtime)."""

__version__ = "0.1.0"
