from .linear import Linear4bit
from .quantization import Quantizer, SymQuantizer
from .hadamard import OnlineHadamard, HadamardQuantizer, fuse_online_hadamard
from .normalization import RMSNorm
from .moe import SignRotMoEBlock
