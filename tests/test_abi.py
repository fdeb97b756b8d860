"""The C-ABI library without a GPU: it loads, exports every entry point that
include/race_attention.h declares, and validates arguments on the host
(no compute call is made)."""
import ctypes
import os
import re

import pytest

from race_attention_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "race_attention.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(race_\w+)\s*\(", text)))


def test_binding_declares_the_header_abi_version():
    m = re.search(r"#define RACE_ABI_VERSION (\d+)", open(HEADER).read())
    assert m and int(m.group(1)) == _lib.ABI_VERSION


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("race_op_fwd", "race_op_bwd", "race_qkv_fwd", "race_qkv_bwd", "race_decode_step",
                 "race_soft_hash_fwd", "race_soft_hash_bwd", "race_qkv_final_state"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in race_attention.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_sizes():
    lib = _lib.load_library()
    assert lib.race_abi_version() == 2 == _lib.ABI_VERSION
    sh = _lib.QKVShape(1, 4, 4, 1 << 20, 64, 8, 4, 8.0, 1e-6, 0)
    state = lib.race_qkv_state_bytes(sh)
    # per-block states (A and St, fp32, one slot per block plus the final state), not [T,S]
    # probabilities: a whole number of (S, D+1) slots for each of the Z = 4 streams
    slot = 4 * 128 * (64 + 1) * 4
    nslots = round(state / slot)
    assert abs(state - nslots * slot) < 512 and 2 <= nslots <= (1 << 20) // 256 + 1
    assert state < 0.02 * 2 * 4 * (1 << 20) * 128 * 4
    assert lib.race_qkv_scratch_bytes(sh, 0) == 0  # S = 128 fits one bucket tile
    assert lib.race_qkv_scratch_bytes(sh, 1) >= state
    assert lib.race_op_workspace_bytes(16, 2048, 128, 64, 0, 1) > 0


@pytest.mark.parametrize("shape,msg", [
    ((1, 4, 3, 128, 64, 8, 4), "multiple"),      # Hq not a multiple of Hkv
    ((1, 4, 4, 128, 96, 8, 4), "head dim"),      # D not compiled in the fused path
    ((1, 4, 4, 128, 64, 8, 5), "K = 5"),         # K > 4
    ((1, 4, 4, (1 << 30) + 1, 64, 8, 4), "2^30"),  # token indices beyond 32-bit headroom
])
def test_qkv_validation_errors(shape, msg):
    lib = _lib.load_library()
    sh = _lib.QKVShape(*shape, 8.0, 1e-6, 0)
    t = _lib.Tensor4(16, 0, 0, 0)
    rc = lib.race_qkv_fwd(sh, t, t, t, ctypes.c_void_p(16), t, 1, ctypes.c_void_p(16), 1 << 30,
                          None, 0, None)
    assert rc != 0
    assert msg in lib.race_last_error().decode()


def test_workspace_too_small_is_reported():
    lib = _lib.load_library()
    rc = lib.race_op_fwd(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                         2, 100, 24, 64, 1e-6, 0, ctypes.c_void_p(16), 8, None)
    assert rc == 3 and "workspace" in lib.race_last_error().decode()


def test_misaligned_bf16_rows_rejected():
    lib = _lib.load_library()
    sh = _lib.QKVShape(1, 2, 2, 64, 64, 8, 4, 8.0, 1e-6, 0)
    bad = _lib.Tensor4(16 + 2, 64 * 64, 64 * 64, 64)
    good = _lib.Tensor4(16, 2 * 64 * 64, 64 * 64, 64)
    rc = lib.race_qkv_fwd(sh, bad, good, good, ctypes.c_void_p(16), good, 1, ctypes.c_void_p(16), 1 << 30,
                          None, 0, None)
    assert rc == 1 and "aligned" in lib.race_last_error().decode()
    # a token stride beyond the row movers' 24-bit offset multiply is refused, not wrapped
    wide = _lib.Tensor4(16, 0, 0, 1 << 24)
    rc = lib.race_qkv_fwd(sh, good, wide, good, ctypes.c_void_p(16), good, 1, ctypes.c_void_p(16), 1 << 30,
                          None, 0, None)
    assert rc == 2 and "token stride" in lib.race_last_error().decode()


def test_cpu_tensors_rejected_without_fallback():
    import torch

    from race_attention_amd import RaceCausalFn
    x = torch.rand(1, 8, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        RaceCausalFn.apply(x, x, torch.rand(1, 8, 16), 1e-6)


def test_kept_state_must_be_aligned():
    lib = _lib.load_library()
    assert lib.race_op_state_bytes(2, 100, 24, 64, 0) > 0
    assert lib.race_op_state_bytes(0, 100, 24, 64, 0) == 0
    rc = lib.race_op_fwd_keep(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                              2, 100, 24, 64, 1e-6, 0, ctypes.c_void_p(16), 1 << 30, ctypes.c_void_p(256 + 4), 1 << 30,
                              None)
    assert rc == 1 and "256-byte aligned" in lib.race_last_error().decode()
    rc = lib.race_op_bwd_kept(*(ctypes.c_void_p(16),) * 7, 2, 100, 24, 64, 1e-6, 0, ctypes.c_void_p(16), 1 << 30,
                              None, 1 << 30, None)
    assert rc == 1 and "256-byte aligned" in lib.race_last_error().decode()


def test_nc_view_arguments_are_checked():
    """race_nc_fwd_view / race_nc_bwd_view reject, on the host, bad stream counts, null views and
    token strides below D, and check a given state's size as the kept entry points do."""
    lib = _lib.load_library()
    p = ctypes.c_void_p(256)
    ok = _lib.Tensor4(256, 4 * 4096 * 64, 4096 * 64, 64)
    ws = (ctypes.c_void_p(256), 1 << 30)
    err = lambda: lib.race_last_error().decode()
    assert lib.race_nc_fwd_view(p, p, ok, ok, 0, 4, 4096, 24, 64, 1e-6, 0, *ws, None, 0, None) == 1
    assert "B and H must be positive" in err()
    short = _lib.Tensor4(256, 0, 0, 32)
    assert lib.race_nc_fwd_view(p, p, short, ok, 2, 4, 4096, 24, 64, 1e-6, 0, *ws, None, 0, None) == 1
    assert "token stride" in err()
    null = _lib.Tensor4(0, 0, 0, 64)
    assert lib.race_nc_fwd_view(p, p, ok, null, 2, 4, 4096, 24, 64, 1e-6, 0, *ws, None, 0, None) == 1
    assert "null out" in err()
    assert lib.race_nc_bwd_view(p, p, ok, ok, p, p, null, 2, 4, 4096, 24, 64, 1e-6, 0, *ws, None, 0, None) == 1
    assert "null gV" in err()
    small = lib.race_op_state_bytes(8, 1024, 24, 64, 0)
    assert lib.race_nc_bwd_view(p, p, ok, ok, p, p, ok, 2, 4, 4096, 24, 64, 1e-6, 0, *ws, ctypes.c_void_p(512),
                                small, None) == 3
    assert "state of" in err()


KEPT = [("race_op_fwd_keep", 4), ("race_op_bwd_kept", 7), ("race_nc_op_fwd_keep", 4), ("race_nc_op_bwd_kept", 7),
        ("race_causal_dot_product_keep", 4), ("race_causal_dot_backward_kept", 7)]


@pytest.mark.parametrize("name,nptr", KEPT)
def test_kept_state_size_is_checked(name, nptr):
    """Every kept-state entry point rejects, on the host, a state buffer smaller than its own
    geometry needs (one sized for a shorter sequence or another block), before any launch."""
    lib = _lib.load_library()
    fn = getattr(lib, name)
    linear = "dot" in name
    need = lib.race_op_state_bytes(2, 4096, 24, 64, 0)
    small = lib.race_op_state_bytes(2, 1024, 24, 64, 0)
    assert 0 < small < need
    ptrs = (ctypes.c_void_p(256),) * nptr
    head = (2, 4096, 24, 64) + (() if linear else (1e-6,)) + (0, ctypes.c_void_p(256), 1 << 30)
    for bytes_, ok in ((small, False), (need - 1, False)):
        rc = fn(*ptrs, *head, ctypes.c_void_p(512), bytes_, None)
        assert rc == 3 and "state of" in lib.race_last_error().decode(), (name, bytes_)
    # a buffer sized for another block (128 tokens: fewer block slots than the automatic 64)
    other = lib.race_op_state_bytes(2, 4096, 24, 64, 128)
    assert 0 < other < need
    assert fn(*ptrs, *head, ctypes.c_void_p(512), other, None) == 3


def test_op_state_raises_the_geometry_error():
    """op_state / linear_state raise the library's reason when the geometry is rejected (here a
    head dim beyond the compiled 256) instead of handing on an empty buffer."""
    import torch
    from race_attention_amd.race_causal_cuda import op_state
    with pytest.raises(_lib.RaceError, match="head dim"):
        op_state(torch.empty(1, 8, 24), torch.empty(1, 8, 300))


@pytest.mark.parametrize("B,Hq,Hkv,T,D,L,Kb", [(1, 4, 4, 1 << 20, 64, 8, 4), (4, 16, 16, 65536, 64, 16, 4),
                                               (1, 8, 2, 1 << 18, 64, 8, 4), (1, 4, 4, 1 << 24, 64, 8, 4),
                                               (2, 4, 1, 333, 128, 3, 3), (1, 2, 2, 65536, 64, 8, 4)])
def test_full_size_tests_know_the_block_geometry(B, Hq, Hkv, T, D, L, Kb):
    """tests/race_ref.qkv_blocks (where the full-size GPU tests put their block-boundary windows)
    agrees with the library: the state it sizes holds exactly NB + 1 slots per stream and tile."""
    import sys
    sys.path.insert(0, os.path.dirname(__file__))
    from race_ref import qkv_blocks
    lib = _lib.load_library()
    sh = _lib.QKVShape(B, Hq, Hkv, T, D, L, Kb, 8.0, 1e-6, 0)
    CB, NB = qkv_blocks(T, B * Hkv, L, Kb, D)
    S = L << Kb
    st = next((x for x in (32, 64, 128) if (128 if D == 64 else 64) >= x >= S), 128 if D == 64 else 64)
    S_pad = -(-S // st) * st
    slots = B * Hkv * (NB + 1) * S_pad
    a256 = lambda n: (n + 255) // 256 * 256
    assert lib.race_qkv_state_bytes(sh) == a256(slots * D * 4) + a256(slots * 4)
    assert (NB - 1) * CB < T <= NB * CB and CB % 32 == 0


def test_qkv_bwd_static_refuses_oversize_on_the_host():
    """race_qkv_bwd_static checks the shape's backward scratch against its static array on the
    host before any HIP call: S = 256 at D = 64 (two bucket tiles' partial outputs) is refused."""
    lib = _lib.load_library()
    assert lib.race_static_scratch_bytes() == 32 << 20
    sh = _lib.QKVShape(1, 2, 2, 65536, 64, 16, 4, 8.0, 1e-6, 0)
    assert lib.race_qkv_scratch_bytes(sh, 1) > lib.race_static_scratch_bytes()
    t = _lib.Tensor4(256, 0, 0, 64)
    rc = lib.race_qkv_bwd_static(sh, t, t, t, t, ctypes.c_void_p(256), ctypes.c_void_p(256), 1 << 40, t, t, t, None)
    assert rc == 3 and "beyond the static" in lib.race_last_error().decode()
    # cfg3 (B=1, H=4, T=2^20) and cfg5's layer (B=8, 32/8 heads, T=8192) fit the array
    for shape in ((1, 4, 4, 1 << 20, 64, 8, 4), (8, 32, 8, 8192, 64, 8, 4)):
        s2 = _lib.QKVShape(*shape, 8.0, 1e-6, 0)
        assert 0 < lib.race_qkv_scratch_bytes(s2, 1) <= lib.race_static_scratch_bytes()


def test_nc_view_layouts_need_no_copy():
    """BatchedACE's [M,B,T,H,d] values reach race_nc_*_view as [M*B, H, T, d] views of the same
    storage (no permute copy); where the strides allow no such view (an expanded ensemble axis) the
    helper says so and the caller copies."""
    import torch
    from race_attention_amd.noncausal import _bhtd
    x = torch.randn(2, 3, 5, 4, 8)
    v = _bhtd(x)
    assert v.shape == (6, 4, 5, 8) and v.data_ptr() == x.data_ptr() and v.stride(3) == 1
    assert torch.equal(v, x.permute(0, 1, 3, 2, 4).reshape(6, 4, 5, 8))
    # the [B,H,T,D] wrapper's M = 1 pack (race_attention): a view of the caller's tensor
    q = torch.randn(3, 4, 5, 8)
    p1 = q.permute(0, 2, 1, 3).unsqueeze(0).expand(1, -1, -1, -1, -1)
    assert _bhtd(p1).data_ptr() == q.data_ptr()
    # M = 2 copies of one tensor (stride 0 on M): no view
    p2 = q.permute(0, 2, 1, 3).unsqueeze(0).expand(2, -1, -1, -1, -1)
    assert _bhtd(p2) is None
    # the upstream gradient of out.sum(dim=2) is expanded along T (token stride 0): _bhtd gives a
    # view with stride 0, _bhtd_rows copies it to distinct rows with the same values
    from race_attention_amd.noncausal import _bhtd_rows
    g = torch.randn(2, 3, 1, 4, 8).expand(2, 3, 5, 4, 8)
    assert _bhtd(g).stride(2) == 0
    r = _bhtd_rows(g)
    assert r.stride(2) >= 8 and r.stride(1) > 0 and torch.equal(r, g.permute(0, 1, 3, 2, 4).reshape(6, 4, 5, 8))
    assert _bhtd_rows(x).data_ptr() == x.data_ptr()  # distinct rows already: no copy


@pytest.mark.parametrize("out_strides", [
    (3 * 100 * 64, 0, 64),       # every head writes the same rows
    (0, 100 * 64, 64),           # every stream writes the same rows
    (3 * 100 * 64, 64, 64),      # head and token strides both D: token t of head h is token t+1 of h-1
])
def test_noncausal_view_rejects_overlapping_outputs(out_strides):
    """race_nc_fwd_view / race_nc_bwd_view refuse an output view (out, gV) whose rows of different
    (stream, head, token) overlap: concurrent workgroups would race on them. Inputs may share rows
    (here one row set read by every stream). The refusal is the host-side argument check, made
    before any launch."""
    lib = _lib.load_library()
    Bz, H, T, S, D = 2, 3, 100, 24, 64
    shared_in = _lib.Tensor4(256, 0, 0, 64)
    bad = _lib.Tensor4(256, *out_strides)
    fake = ctypes.c_void_p(256)
    rc = lib.race_nc_fwd_view(fake, fake, shared_in, bad, Bz, H, T, S, D, 1e-6, 0, fake, 1 << 40, None, 0, None)
    assert rc == 1 and "overlapping" in lib.race_last_error().decode()
    rc = lib.race_nc_bwd_view(fake, fake, shared_in, shared_in, fake, fake, bad, Bz, H, T, S, D, 1e-6, 0, fake,
                              1 << 40, None, 0, None)
    assert rc == 1 and "overlapping" in lib.race_last_error().decode()


def test_integration_bindings_match_the_library_signatures():
    """The ctypes stubs that INTEGRATION.md shows a maintainer of the reference declare the same
    argument types as the package's own binding (which the header test above pins)."""
    import ctypes
    text = open(os.path.join(os.path.dirname(HEADER), "..", "INTEGRATION.md")).read()
    alias = {"vp": ctypes.c_void_p, "c_void_p": ctypes.c_void_p, "i64": ctypes.c_int64,
             "c_int64": ctypes.c_int64, "f32": ctypes.c_float, "c_float": ctypes.c_float,
             "c_int": ctypes.c_int, "c_size_t": ctypes.c_size_t, "Tensor4": _lib.Tensor4}
    found = re.findall(r"\b_?lib\.(race_\w+)\.argtypes = \[([^\]]*)\]", text, flags=re.S)
    assert len(found) >= 4
    for name, args in found:
        got = [alias[a.strip().replace("ctypes.", "")] for a in args.split(",") if a.strip()]
        assert got == list(_lib.SIGNATURES[name][1]), name
    for name, res in re.findall(r"\b_?lib\.(race_\w+)\.restype = ([\w.]+)", text):
        assert alias.get(res.replace("ctypes.", ""), getattr(ctypes, res.replace("ctypes.", ""), None)) \
            == _lib.SIGNATURES[name][0], name
