"""blog_amd: MI355X (gfx950) GGUF quantized-linear hot path.

The product is ``libqlin.so`` (HIP kernels behind the C ABI in ``include/qlin.h``); ``blog_amd.qlin``
is its ctypes binding and ``blog_amd.build`` its gfx950 build.
"""
