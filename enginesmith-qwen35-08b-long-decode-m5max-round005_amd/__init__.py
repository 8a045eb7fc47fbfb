"""MI355X-native batch-1 long-context decode engine for the Qwen3.5-0.8B-shape
hybrid model (Q4 weights): HIP kernels for gfx950 and a C++ engine behind the
C ABI in include/es_decode.h, built into libesdecode.so. `esdecode` is the
ctypes binding; it raises if the library has not been built."""
from .esdecode import *  # noqa: F401,F403
from .esdecode import lib, LIB_PATH, SERVER_PATH  # noqa: F401
