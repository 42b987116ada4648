from .linear import Linear4bit, AsymSymmLinear4bit
from .quantization import Quantizer, SymQuantizer, AsymQuantizer
from .hadamard import OnlineHadamard, HadamardQuantizer, fuse_online_hadamard
from .normalization import RMSNorm
from .moe import SignRotMoEBlock
