"""MI355X (gfx950) attention path for voxtral.cpp.

GGML_OP_FLASH_ATTN_EXT behind a C ABI (include/vxfa.h, libvxfa.so):
`vxfa` is the ctypes binding, `views` the tensor layouts voxtral.cpp uses.
The directory name is not a Python identifier; load it with load_package().
"""
from . import views, vxfa  # noqa: F401
