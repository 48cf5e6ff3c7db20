"""mindpipe_amd: MI355X (gfx950) quantized-linear forward path for MindPipe.

Drop-in replacements for the reference's quantized-linear module API backed by
hand-written HIP kernels behind a C ABI (``include/mindpipe_amd.h``).
"""
__version__ = "0.1.0"
