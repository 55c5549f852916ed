"""MI355X-native backend for 0xBitNet's ternary inference path.

The compute path is liboxbitnet.so (hand-written HIP for gfx950 behind the
0xBitNet C ABI); this package is its Python binding:

    BitNet   - the reference's Python API (load_sync / generate / chat / ...)
    Model    - ids-level engine: forward(ids), greedy decode as hipGraph replays
    Batch    - batched greedy decode of independent sequences on a Model
    ops      - the individual hot-path kernels (numpy in, numpy out)
    synth    - synthetic random-init BitNet GGUF files
"""
from ._native import LIB_PATH, NativeError, lib
from .bitnet import Batch, BitNet, Model

__all__ = ["Batch", "BitNet", "Model", "NativeError", "lib", "LIB_PATH"]
__version__ = "0.1.0"
