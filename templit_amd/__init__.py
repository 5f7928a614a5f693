"""templit_amd: an MI355X-native runtime backend for TempLit.

The product is native code:
  * libtemplit_hip.so -- hand-written gfx950 HIP kernels behind the C-ABI of
    include/templit_hip.h;
  * hip::Runtime / Storage<hip::HIP, T> (templit_amd/include/my_hip/) -- the
    C++ host runtime with the operation surface passes::Compiled dispatches
    through, calling only that C-ABI;
  * libtemplit_gpt.so -- the GPT training-step program (include/templit_gpt.h).

This Python package only locates and binds those libraries (native.py) and
builds them (build.py).
"""
from .native import GPT_LIB, HIP_LIB, NativeError, load_hip  # noqa: F401
