"""perseus_amd: an MI355X (gfx950) engine for the CKKS key-switch / NTT path of gladia-research-group/perseus.

libpchip.so holds the hand-written HIP kernels behind the reference's KernelTable ABI (include/pc_hip.h), the HIP
runtime FFI and the key-switching driver; this package binds them.
"""
from ._lib import LIB, HipError, check, header_functions  # noqa: F401
from .chains import Chain, preset  # noqa: F401
from .chains import make as make_chain  # noqa: F401
from .engine import Context, Decryptor, DevBuf, Drbg, Event, Graph, Keys, Rows, Stream, device_count, ntt_one_pass_min  # noqa: F401
