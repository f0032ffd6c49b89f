"""krunch_amd: MI355X (gfx950) engine for krunch's batched RWKV-4 compress/decompress path.

Modules mirroring the reference's interfaces:
  krunch_amd.krunch_ac       <- krunch_ac (probs_to_cdf, encode, decode)
  krunch_amd.krunch_ac_hip   <- the krunch_ac_cuda extension ops
  krunch_amd.cpp_path        <- krunch.cpp_path
  krunch_amd.batched_rwkv4   <- krunch.batched_rwkv4
  krunch_amd.inference       <- krunch.inference (engine, blob header)
All compute goes through libkrunch_hip.so (C ABI: include/krunch_hip.h).
"""
__version__ = "0.1.0"
