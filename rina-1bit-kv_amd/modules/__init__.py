"""KVR on MI355X: drop-in `modules` package (WindowBuffer, RetrievalIndex, KVRHook, KVRGenerator)
backed by the gfx950 HIP kernels of libkvr_hip.so (see _hip.py)."""
