"""ctypes binding of libkrunch_hip.so (the C ABI declared in include/krunch_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in the product. If
the library is missing, build it with `python -m krunch_amd.build`.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkrunch_hip.so")

P = ctypes.c_void_p
I = ctypes.c_int
LL = ctypes.c_longlong
U32 = ctypes.c_uint32
SZ = ctypes.c_size_t


class KrPackedJob(ctypes.Structure):
    _fields_ = [("xf", P), ("Wf", P), ("N", I), ("out", P), ("ldo", LL), ("epilogue", I),
                ("res", P), ("gate", P), ("out_packed", I)]


class KrMatrixQ8(ctypes.Structure):
    _fields_ = [("q", P), ("qf", P), ("scale", P)]


class KrLayerQ8(ctypes.Structure):
    _fields_ = [(n, KrMatrixQ8) for n in ("K", "V", "R", "O", "fK", "fV", "fR")]


class KrLayerWeights(ctypes.Structure):
    _fields_ = [(n, P) for n in (
        "ln1_w", "ln1_b", "tm_k", "tm_v", "tm_r", "decay", "first",
        "Kt", "Vt", "Rt", "Ot", "ln2_w", "ln2_b", "ftm_k", "ftm_r", "fKt", "fVt", "fRt",
        "Kf", "Vf", "Rf", "Of", "fKf", "fVf", "fRf")] + [("q8", ctypes.POINTER(KrLayerQ8))]


class KrModelWeights(ctypes.Structure):
    _fields_ = [("n_layer", I), ("C", I), ("F", I), ("V", I), ("emb", P),
                ("ln_out_w", P), ("ln_out_b", P), ("headT", P),
                ("layers", ctypes.POINTER(KrLayerWeights)), ("headF", P)]


# name -> (argtypes, restype); every int-returning entry point is checked.
_SIGS = {
    "kr_last_error": ([], ctypes.c_char_p),
    "kr_abi_version": ([], I),
    # range coder
    "kr_encode_step": ([P, I, P, I, P, U32, P, I, P, P], I),
    "kr_encode_finalize": ([P, U32, P, P, P], I),
    "kr_encode_step_batched": ([P, I, P, P, U32, P, P, I, I, P, P], I),
    "kr_encode_pairs_batched": ([P, I, LL, P, P, U32, P, P, I, I, P, P], I),
    "kr_encode_finalize_batched": ([P, U32, P, P, I, P, P], I),
    "kr_decode_init_batched": ([P, U32, P, P, P, I, P], I),
    "kr_decode_step_batched": ([P, I, P, U32, P, P, P, P, I, I, P], I),
    # CDF
    "kr_probs_to_cdf": ([P, I, I, LL, P, I, P], I),
    "kr_softmax_cdf": ([P, I, I, LL, P, I, I, P], I),
    "kr_softmax_probs": ([P, I, I, LL, P, P], I),
    "kr_softmax_cdf_pairs": ([P, I, I, LL, P, P, I, P], I),
    "kr_softmax_cdf_decode": ([P, I, I, LL, P, U32, P, P, P, P, P, LL, P, P, I, P], I),
    # GEMM / layers / model
    "kr_transpose_f16": ([P, LL, I, I, P, LL, P], I),
    "kr_det_matmul": ([P, I, I, P, LL, I, P, LL, I, P, P, P], I),
    "kr_fragment_bytes": ([I, I], ctypes.c_size_t),
    "kr_pack_fragments": ([P, LL, I, I, P, P], I),
    "kr_det_matmul_packed": ([P, I, I, P, I, P, LL, I, P, P, I, P], I),
    "kr_det_matmul_packed_multi": ([ctypes.POINTER(KrPackedJob), I, I, I, P], I),
    "kr_quant_bytes": ([I, I, I], ctypes.c_size_t),
    "kr_quantize_rows": ([P, LL, I, I, P, P, I, P], I),
    "kr_det_matmul_i8": ([P, P, I, I, P, P, I, P, LL, I, P, P, I, P], I),
    "kr_prepare_decay": ([P, P, I, P], I),
    "kr_state_bytes": ([I, I, I], SZ),
    "kr_state_init": ([P, I, I, I, P], I),
    "kr_forward_workspace_bytes": ([LL, I, I], SZ),
    "kr_layer_step": ([ctypes.POINTER(KrLayerWeights), I, I, P, I, I, P, P, P, P, P, P, SZ, P], I),
    "kr_layer_step_noalloc": ([ctypes.POINTER(KrLayerWeights), I, I, P, I, I, P, P, P, P, P, P],
                              I),
    "kr_wkv": ([I, I, I, P, P, P, P, P, P, P, P, P, P], I),
    "kr_phase_profile": ([I], I),
    "kr_phase_count": ([], I),
    "kr_phase_name": ([I], ctypes.c_char_p),
    "kr_read_phase_times": ([ctypes.POINTER(ctypes.c_double), I, ctypes.POINTER(LL)], I),
    "kr_reset_phase_times": ([], I),
    "kr_step_timing": ([I, ctypes.POINTER(I)], I),
    "kr_step_timing_read": ([ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double), I,
                             ctypes.POINTER(I)], I),
    "kr_forward_layers": ([ctypes.POINTER(KrModelWeights), P, I, I, P, P, SZ, P], I),
    "kr_embed": ([ctypes.POINTER(KrModelWeights), P, I, P, P], I),
    "kr_head_logits": ([ctypes.POINTER(KrModelWeights), P, I, P, P, LL, P], I),
    "kr_compress_window": ([ctypes.POINTER(KrModelWeights), P, P, I, I, P, P, P, SZ, P, LL, I,
                            P, I, P], I),
    "kr_decode_step": ([ctypes.POINTER(KrModelWeights), I, P, P, P, P, SZ, P, LL, P, U32, P, P,
                        P, P, LL, P, P, I, P], I),
    "kr_decode_workspace_bytes": ([I, I, I, I], SZ),
    "kr_decode_run": ([ctypes.POINTER(KrModelWeights), I, P, P, P, P, SZ, P, LL, P, U32, P, P,
                       P, P, LL, P, P, I, I, I, I, P], I),
}

_lib = None


class KrunchError(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run `python -m krunch_amd.build` "
                              "(the HIP library is required: there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGS)


def call(name: str, *args):
    """Call an int-returning entry point and raise KrunchError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().kr_last_error().decode(errors="replace")
        raise KrunchError(f"{name} failed ({rc}): {msg}")
    return rc


NOALLOC_SCRATCH_BYTES = 32 << 20      # KR_NOALLOC_SCRATCH_BYTES of include/krunch_hip.h
U32_MAX = 0xFFFFFFFF
I32_MAX = 0x7FFFFFFF


def u32(n: int, what: str = "size") -> int:
    """A byte count passed as uint32_t: ctypes would truncate silently, so
    anything outside [0, 2^32) is an error here."""
    n = int(n)
    if n < 0 or n > U32_MAX:
        raise ValueError(f"{what} = {n} does not fit the 32-bit coder interface "
                         f"(split the call so it stays <= {U32_MAX})")
    return n


def ptr(t) -> int | None:
    """Raw device pointer of a torch tensor (None stays NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(stream=None) -> int | None:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream
