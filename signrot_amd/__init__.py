"""MI355X-native (gfx950) SignRot W4A4 real-quant path.

Drop-in for the reference's `signrot` package on its hot path: the module
API (`signrot_amd.nn`, `signrot_amd.functional`) mirrors `signrot.nn` /
`signrot.functional`, and `signrot_amd._CUDA` mirrors the `signrot._CUDA`
op table, backed by hand-written HIP kernels in
signrot_amd/_lib/libsignrot_hip.so (C ABI: include/signrot_hip.h).
"""
from . import functional
from . import nn
