"""KVR on MI355X: drop-in `modules` package (WindowBuffer, RetrievalIndex, KVRHook, KVRGenerator)
backed by the gfx950 HIP kernels of libkvr_hip.so (see _hip.py)."""
from .kvr_window import WindowBuffer
from .kvr_retrieval import RetrievalIndex
from .kvr_cache import TileKVCache
from .kvr_hook import KVRHook
from .kvr_generator import KVRGenerator

__all__ = ["WindowBuffer", "RetrievalIndex", "TileKVCache", "KVRHook", "KVRGenerator"]
