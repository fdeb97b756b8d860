"""race_qkv_bwd_static (the fused backward with its scratch in a static device array, for callers
that cannot allocate) against race_qkv_bwd with a caller's workspace, through the C ABI: bitwise
the same dq, dk, dv on two calls in a row, the second on a smaller input (the array keeps the
first call's contents), and no allocation through torch's allocator during the call."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _views(lib_mod, *ts):
    return [lib_mod.view4(t)[0] for t in ts]


@pytest.mark.parametrize("order", ["large_then_small"])
def test_qkv_bwd_static_equals_workspace_entry_point(dev, order):
    from race_attention_amd import _lib, build_planes_protos
    lib = _lib.lib()
    cases = [(2, 8, 4, 3000, 64, 8, 4), (1, 4, 2, 700, 64, 8, 4)]  # the second is smaller
    for (B, Hq, Hkv, T, D, L, Kb) in cases:
        print(f"static-scratch backward B={B} Hq={Hq} Hkv={Hkv} T={T} D={D} L={L} K={Kb}", flush=True)
        planes = build_planes_protos(D, Kb, L, 1, device=dev, seed=3)[0].contiguous()
        g = torch.Generator(device=dev).manual_seed(T)
        q = torch.randn(B, Hq, T, D, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(B, Hkv, T, D, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(B, Hkv, T, D, generator=g, device=dev).to(torch.bfloat16)
        go = torch.randn(B, Hq, T, D, generator=g, device=dev).to(torch.bfloat16)
        sh = _lib.QKVShape(B, Hq, Hkv, T, D, L, Kb, math.sqrt(D), 1e-6, 0)
        need = lib.race_qkv_scratch_bytes(sh, 1)
        assert 0 < need <= lib.race_static_scratch_bytes()
        state = _lib.workspace(lib.race_qkv_state_bytes(sh), dev)
        fscr = _lib.workspace(lib.race_qkv_scratch_bytes(sh, 0), dev)
        out = torch.empty(B, Hq, T, D, dtype=torch.bfloat16, device=dev)
        s = _lib.stream_of(q)
        qv, kv, vv, gv, ov = _views(_lib, q, k, v, go, out)
        _lib.check(lib.race_qkv_fwd(sh, qv, kv, vv, _lib.ptr(planes), ov, _lib.RACE_BF16, _lib.ptr(state),
                                    state.numel(), _lib.ptr(fscr), fscr.numel(), s), "race_qkv_fwd")
        ref = [torch.empty_like(t) for t in (q, k, v)]
        scr = _lib.workspace(need, dev)
        rv = _views(_lib, *ref)
        _lib.check(lib.race_qkv_bwd(sh, qv, kv, vv, gv, _lib.ptr(planes), _lib.ptr(state), state.numel(), *rv,
                                    _lib.ptr(scr), scr.numel(), s), "race_qkv_bwd")
        got = [torch.full_like(t, float("nan")) for t in (q, k, v)]
        gvv = _views(_lib, *got)
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(dev)
        _lib.check(lib.race_qkv_bwd_static(sh, qv, kv, vv, gv, _lib.ptr(planes), _lib.ptr(state), state.numel(),
                                           *gvv, s), "race_qkv_bwd_static")
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == before
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert torch.equal(a, b), f"{name} of the static-scratch backward differs (T={T})"


# The refusal of shapes beyond the static array is a host-side check, tested without a GPU in
# tests/test_abi.py (test_qkv_bwd_static_refuses_oversize_on_the_host).
