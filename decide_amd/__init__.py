"""MI355X (gfx950) encoder forward for jmwri/decide.

The product is libdecide_hip.so (C ABI: include/decide_hip.h, sources in
csrc/). This package is a thin ctypes veneer over it for tests, the bench and
Python callers: nn (Config, Sequence, build_sequence, Engine), local (question
types, PackText, Local with one batched forward per SystemOne call, answer
post-processing), bundle (safetensors and bundle loading, BF16 included) and
synth (seeded benchmark inputs).
"""
from .nn import (CLS_ID, MASK_ID, SEP_ID, Config, Engine, Sequence, build_sequence, config_from_dict,  # noqa: F401
                 load_config, modernbert_base, open_engine, tensor_shapes)
from .native import DecideError, InvalidArgument, NoGPUError, Unsupported  # noqa: F401
