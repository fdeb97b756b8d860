"""ctypes bindings for oracle/liborace.so -- TEST INFRASTRUCTURE ONLY.

Wraps the C restatements in race_pref_oracle.c (see that file's header for the
reference file:line each one follows). Used by tests/, smoke() and bench.py's
cpu_baseline leg as the checker; the HIP product never imports this module.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liborace.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(path)
        i64, dbl, vp = ctypes.c_int64, ctypes.c_double, ctypes.c_void_p
        L.orc_prefix_mean_flat.argtypes = [vp, vp, vp, i64, i64, i64, dbl]
        L.orc_prefix_mean_flat_bw.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, dbl]
        L.orc_race_fwd.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, dbl]
        L.orc_race_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, dbl]
        L.orc_race_windows.argtypes = [vp, vp, vp, vp, i64, i64, i64, dbl, vp, vp, vp, i64, i64,
                                       vp, vp, vp, vp]
        for f in (L.orc_prefix_mean_flat, L.orc_prefix_mean_flat_bw, L.orc_race_fwd, L.orc_race_bwd,
                  L.orc_race_windows):
            f.restype = None
        _LIB = L
    return _LIB


def _c(t, dtype):
    t = t.detach().to("cpu", dtype).contiguous()
    return t, ctypes.c_void_p(t.data_ptr())


def prefix_mean_flat(w, v, eps):
    """E[NS,T,D] from w[NS,T], v[NS,T,D] (fp32), as race_pref.cpp:36-101."""
    w, pw = _c(w, torch.float32)
    v, pv = _c(v, torch.float32)
    NS, T, D = v.shape
    E = torch.empty(NS, T, D, dtype=torch.float32)
    lib().orc_prefix_mean_flat(pw, pv, ctypes.c_void_p(E.data_ptr()), NS, T, D, float(eps))
    return E


def prefix_mean_flat_bw(w, v, gE, eps):
    """(gW[NS,T], gV[NS,T,D]) as race_pref.cpp:104-220."""
    w, pw = _c(w, torch.float32)
    v, pv = _c(v, torch.float32)
    gE, pg = _c(gE, torch.float32)
    NS, T, D = v.shape
    gW = torch.empty(NS, T, dtype=torch.float32)
    gV = torch.empty(NS, T, D, dtype=torch.float32)
    lib().orc_prefix_mean_flat_bw(pw, pv, pg, ctypes.c_void_p(gW.data_ptr()),
                                  ctypes.c_void_p(gV.data_ptr()), NS, T, D, float(eps))
    return gW, gV


def race_fwd(pK, pQ, V, eps):
    """Streaming fp64 causal RACE forward: (out[N,T,D], A_final[N,S], B_final[N,S,D])."""
    pK, a = _c(pK, torch.float64)
    pQ, b = _c(pQ, torch.float64)
    V, c = _c(V, torch.float64)
    N, T, S = pK.shape
    D = V.shape[2]
    out = torch.empty(N, T, D, dtype=torch.float64)
    Af = torch.empty(N, S, dtype=torch.float64)
    Bf = torch.empty(N, S, D, dtype=torch.float64)
    lib().orc_race_fwd(a, b, c, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(Af.data_ptr()),
                       ctypes.c_void_p(Bf.data_ptr()), N, T, S, D, float(eps))
    return out, Af, Bf


def race_bwd(pK, pQ, V, gO, eps):
    """Streaming fp64 exact backward: (gpK[N,T,S], gpQ[N,T,S], gV[N,T,D])."""
    pK, a = _c(pK, torch.float64)
    pQ, b = _c(pQ, torch.float64)
    V, c = _c(V, torch.float64)
    gO, d = _c(gO, torch.float64)
    N, T, S = pK.shape
    D = V.shape[2]
    gpK = torch.empty(N, T, S, dtype=torch.float64)
    gpQ = torch.empty(N, T, S, dtype=torch.float64)
    gV = torch.empty(N, T, D, dtype=torch.float64)
    lib().orc_race_bwd(a, b, c, d, ctypes.c_void_p(gpK.data_ptr()), ctypes.c_void_p(gpQ.data_ptr()),
                       ctypes.c_void_p(gV.data_ptr()), N, T, S, D, float(eps))
    return gpK, gpQ, gV


def race_windows(pK, pQ, V, gO, eps, wins, wlen, A0=None, B0=None):
    """One stream (pK, pQ [T,S], V [T,D], gO [T,D] or None) of the streaming fp64 forward
    and backward, kept on the token windows [w, w + wlen) for w in `wins` (sorted, disjoint),
    starting from the carried-in bucket state (A0 [S], B0 [S,D]) when given.
    Returns out [nwin,wlen,D] and, with gO, (gpK, gpQ [nwin,wlen,S], gV [nwin,wlen,D])."""
    pK, a = _c(pK, torch.float64)
    pQ, b = _c(pQ, torch.float64)
    V, c = _c(V, torch.float64)
    T, S = pK.shape
    D = V.shape[1]
    wins = sorted(int(w) for w in wins)
    for i, w in enumerate(wins):
        if w < 0 or w + wlen > T or (i and wins[i - 1] + wlen > w):
            raise ValueError(f"window starts {wins} (length {wlen}) must be disjoint and inside [0, {T})")
    wt = torch.tensor(wins, dtype=torch.int64)
    nw = len(wins)
    out = torch.empty(nw, wlen, D, dtype=torch.float64)
    keep = [pK, pQ, V, wt]
    gp = ctypes.c_void_p(0)
    res = [out]
    if gO is not None:
        gO, gp = _c(gO, torch.float64)
        keep.append(gO)
        res += [torch.empty(nw, wlen, S, dtype=torch.float64), torch.empty(nw, wlen, S, dtype=torch.float64),
                torch.empty(nw, wlen, D, dtype=torch.float64)]
    pa = pb = ctypes.c_void_p(0)
    if A0 is not None:
        A0, pa = _c(A0, torch.float64)
        B0, pb = _c(B0, torch.float64)
        keep += [A0, B0]
    ptrs = [ctypes.c_void_p(r.data_ptr()) for r in res] + [ctypes.c_void_p(0)] * (4 - len(res))
    lib().orc_race_windows(a, b, c, gp, T, S, D, float(eps), pa, pb, ctypes.c_void_p(wt.data_ptr()), nw,
                           int(wlen), *ptrs)
    return res[0] if gO is None else tuple(res)


def _load_ref(name):
    path = os.path.join(_HERE, "_ref", name + ".so")
    if not os.path.exists(path):
        return None
    import importlib.util
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def ref_ext():
    """The reference's own race_pref.cpp compiled into oracle/_ref (None if not built)."""
    return _load_ref("race_pref_ref")


def ref_linear_ext():
    """The reference's own linear_pref.cpp compiled into oracle/_ref (None if not built)."""
    return _load_ref("linear_pref_ref")

