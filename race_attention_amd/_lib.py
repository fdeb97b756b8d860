"""ctypes binding of librace_amd.so (C ABI declared in include/race_attention.h).

Torch is used only as plumbing: device memory (tensors and workspaces from the
caching allocator) and the current HIP stream. Every compute call goes to the
HIP library; there is no CPU or PyTorch fallback. A missing library or a
non-ROCm tensor raises.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librace_amd.so")

RACE_F32 = 0
RACE_BF16 = 1

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class Tensor4(ctypes.Structure):
    """race_tensor: [B][H][T][D] with contiguous last dim, strides in elements."""
    _fields_ = [("data", _vp), ("stride_b", _i64), ("stride_h", _i64), ("stride_t", _i64)]


class HashShape(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("H", ctypes.c_int), ("T", ctypes.c_int), ("D", ctypes.c_int),
                ("L", ctypes.c_int), ("K", ctypes.c_int), ("M", ctypes.c_int),
                ("unshared", ctypes.c_int), ("scale", ctypes.c_float)]


class QKVShape(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("Hq", ctypes.c_int), ("Hkv", ctypes.c_int), ("T", ctypes.c_int),
                ("D", ctypes.c_int), ("L", ctypes.c_int), ("K", ctypes.c_int),
                ("scale", ctypes.c_float), ("eps", ctypes.c_float), ("block", _i64)]


class DecodeShape(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("Hq", ctypes.c_int), ("Hkv", ctypes.c_int), ("D", ctypes.c_int),
                ("L", ctypes.c_int), ("K", ctypes.c_int), ("scale", ctypes.c_float), ("eps", ctypes.c_float)]


# exported symbol -> (restype, argtypes); kept in sync with include/race_attention.h
SIGNATURES = {
    "race_abi_version": (ctypes.c_int, []),
    "race_last_error": (ctypes.c_char_p, []),
    "race_soft_hash_fwd": (ctypes.c_int, [ctypes.POINTER(HashShape), Tensor4, ctypes.c_int, _vp, _vp, _vp]),
    "race_soft_hash_bwd": (ctypes.c_int, [ctypes.POINTER(HashShape), Tensor4, ctypes.c_int, _vp, _vp,
                                          Tensor4, _vp]),
    "race_soft_hash_bwd_partials": (ctypes.c_int, [ctypes.POINTER(HashShape)]),
    "race_soft_hash_bwd_scale": (ctypes.c_int, [ctypes.POINTER(HashShape), Tensor4, ctypes.c_int, _vp, _vp,
                                                Tensor4, _vp, _vp]),
    "race_soft_hash_fwd_dscale": (ctypes.c_int, [ctypes.POINTER(HashShape), Tensor4, ctypes.c_int, _vp, _vp, _vp,
                                                 _vp]),
    "race_soft_hash_bwd_dscale": (ctypes.c_int, [ctypes.POINTER(HashShape), Tensor4, ctypes.c_int, _vp, _vp, _vp,
                                                 Tensor4, _vp, _vp, _vp]),
    "race_nc_op_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64, ctypes.c_int]),
    "race_nc_op_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _i64, _vp,
                                      ctypes.c_size_t, _vp]),
    "race_nc_op_bwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float,
                                      _i64, _vp, ctypes.c_size_t, _vp]),
    "race_nc_op_fwd_keep": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _i64, _vp,
                                           ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_nc_op_bwd_kept": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                           ctypes.c_float, _i64, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_nc_fwd_view": (ctypes.c_int, [_vp, _vp, Tensor4, Tensor4, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                                        _i64, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_nc_bwd_view": (ctypes.c_int, [_vp, _vp, Tensor4, Tensor4, _vp, _vp, Tensor4, _i64, _i64, _i64, _i64, _i64,
                                        ctypes.c_float, _i64, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_causal_dot_product": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp,
                                               ctypes.c_size_t, _vp]),
    "race_causal_dot_backward": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                                _vp, ctypes.c_size_t, _vp]),
    "race_causal_dot_product_keep": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp,
                                                    ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_causal_dot_backward_kept": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                                     _i64, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_op_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64, ctypes.c_int]),
    "race_op_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _i64, _vp,
                                   ctypes.c_size_t, _vp]),
    "race_op_bwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float,
                                   _i64, _vp, ctypes.c_size_t, _vp]),
    "race_op_state_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64]),
    "race_op_fwd_keep": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _i64, _vp,
                                        ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_op_bwd_kept": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float,
                                        _i64, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_qkv_state_bytes": (ctypes.c_size_t, [ctypes.POINTER(QKVShape)]),
    "race_qkv_scratch_bytes": (ctypes.c_size_t, [ctypes.POINTER(QKVShape), ctypes.c_int]),
    "race_qkv_fwd": (ctypes.c_int, [ctypes.POINTER(QKVShape), Tensor4, Tensor4, Tensor4, _vp, Tensor4,
                                    ctypes.c_int, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "race_qkv_bwd": (ctypes.c_int, [ctypes.POINTER(QKVShape), Tensor4, Tensor4, Tensor4, Tensor4, _vp, _vp,
                                    ctypes.c_size_t, Tensor4, Tensor4, Tensor4, _vp, ctypes.c_size_t, _vp]),
    "race_qkv_final_state": (ctypes.c_int, [ctypes.POINTER(QKVShape), _vp, ctypes.c_size_t, _vp, _vp, _vp]),
    "race_static_scratch_bytes": (ctypes.c_size_t, []),
    "race_qkv_bwd_static": (ctypes.c_int, [ctypes.POINTER(QKVShape), Tensor4, Tensor4, Tensor4, Tensor4, _vp, _vp,
                                           ctypes.c_size_t, Tensor4, Tensor4, Tensor4, _vp]),
    "race_decode_step": (ctypes.c_int, [ctypes.POINTER(DecodeShape), _vp, _vp, _vp, ctypes.c_int, _vp, _vp,
                                        _vp, _vp, _vp]),
    "race_profile_enable": (ctypes.c_int, [ctypes.c_int]),
    "race_profile_read": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                         ctypes.POINTER(ctypes.c_int64)]),
    "race_profile_reset": (ctypes.c_int, []),
}

# kernel ids of race_profile_read (include/race_attention.h)
PROF_KERNELS = ["qkv_fwd_totals", "qkv_fwd_readout", "qkv_bwd_totals", "qkv_bwd_main",
                "op_fwd_totals", "op_fwd_readout", "op_bwd_totals", "op_bwd_main",
                "block_scan", "reduce_partials", "softhash_fwd", "softhash_bwd", "decode_step",
                "nc_readout", "nc_backward"]

_LIB = None


# RACE_ABI_VERSION of include/race_attention.h that SIGNATURES declares
ABI_VERSION = 2


def load_library(path=LIB_PATH):
    """Load librace_amd.so and declare every C-ABI signature (no GPU call)."""
    global _LIB
    if _LIB is not None and path == LIB_PATH:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build the HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()' or python -m race_attention_amd._build)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.race_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path} implements C-ABI version {lib.race_abi_version()}, these bindings "
                           f"declare version {ABI_VERSION}: rebuild the library")
    if path == LIB_PATH:
        _LIB = lib
    return lib


def lib():
    return load_library()


class RaceError(RuntimeError):
    pass


def check(rc, what):
    if rc != 0:
        msg = lib().race_last_error().decode(errors="replace")
        raise RaceError(f"{what} failed (status {rc}): {msg}")


def require_device(*tensors):
    for t in tensors:
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise RaceError("race_attention_amd runs on a ROCm GPU: every tensor must be on a "
                            "'cuda' (HIP) device; there is no CPU path")


def stream_of(t):
    return _vp(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t):
    return _vp(t.data_ptr()) if t is not None else _vp(0)


def view4(t):
    """race_tensor of a 4-D [B,H,T,D] tensor whose last dim is contiguous."""
    if t.dim() != 4:
        raise RaceError(f"expected a 4-D [B,H,T,D] tensor, got shape {tuple(t.shape)}")
    if t.stride(3) != 1:
        t = t.contiguous()
    s = t.stride()
    return Tensor4(t.data_ptr(), s[0], s[1], s[2]), t


def dtype_code(dt):
    if dt == torch.float32:
        return RACE_F32
    if dt == torch.bfloat16:
        return RACE_BF16
    raise RaceError(f"unsupported dtype {dt} (float32 or bfloat16)")


def profile(on):
    """Enable/disable per-kernel HIP-event timing inside the library."""
    lib().race_profile_reset()
    lib().race_profile_enable(1 if on else 0)


def profile_read():
    """{kernel name: (total ms, launches)} for every kernel launched since profile(True)."""
    res = {}
    for i, name in enumerate(PROF_KERNELS):
        ms = ctypes.c_double(0.0)
        n = ctypes.c_int64(0)
        check(lib().race_profile_read(i, ctypes.byref(ms), ctypes.byref(n)), "race_profile_read")
        if n.value:
            res[name] = (ms.value, n.value)
    return res


def workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
