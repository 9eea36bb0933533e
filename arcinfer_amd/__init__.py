"""arcinfer_amd: MI355X-native (gfx950) quantized matrix products for GGUF weights -- the quantized matmul path
of arcinferzero (rizagp/arcinfer) as a C-ABI library (include/qmatmul.h, arcinfer_amd/libqmatmul.so) of
hand-written HIP kernels, with a ctypes binding of that ABI (arcinfer_amd.qmatmul) for tests and the bench."""
from . import formats  # noqa: F401
