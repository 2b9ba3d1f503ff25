"""oc_int4_gemm_noalloc (the allocation-free entry point) against
oc_int4_gemm through the C ABI: two calls in a row per layer, the second
with a smaller input, bit for bit equal to the workspace entry point (both
run the same deterministic kernels), plus the scratch-limit error."""
import ctypes

import pytest
import torch

from gpu_helpers import say

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _layer(kind):
    from onecomp_runtime import synthetic
    from onecomp_runtime.layers import FusedInt4LinearPaddedGroups, PackedGPTQLinear

    if kind == "actorder":
        lay = synthetic.gptq_layer(5120, 5120, seed=20600, act_order=True)
        return PackedGPTQLinear(5120, 5120, lay.qweight.to(DEV), lay.scales.to(DEV), lay.qzeros.to(DEV),
                                g_idx=lay.g_idx.to(DEV), groupsize=32)
    lay = synthetic.gptq_layer(1040, 3072, seed=20601, groupsize=26, pad_rows_to=1056)
    return FusedInt4LinearPaddedGroups(1040, 3072, lay.qweight.to(DEV), lay.scales.to(DEV), lay.qzeros.to(DEV),
                                       groupsize=26)


def _call(fn_name, mod, x, out, workspace=None):
    from onecomp_runtime import _hip

    L = _hip.lib()
    w = mod.tiled()
    dt = {torch.bfloat16: _hip.OC_DTYPE_BF16, torch.float16: _hip.OC_DTYPE_F16}
    args = [x.data_ptr(), x.stride(0), dt[x.dtype], x.shape[0], mod.in_features, w.qt.data_ptr(),
            w.st.data_ptr(), dt[w.st.dtype], w.zt.data_ptr(), w.N, w.k_phys, w.group_rows,
            None if mod.kmap is None else mod.kmap.data_ptr(),
            None if mod.kinv is None else mod.kinv.data_ptr(), None, 0, out.data_ptr(), out.stride(0)]
    stream = _hip.stream_of(0)
    if fn_name == "oc_int4_gemm":
        ws, nbytes = workspace
        args += [None if ws is None else ws.data_ptr(), nbytes, 0, stream]
    else:
        args += [0, stream]
    return getattr(L, fn_name)(*args)


@pytest.mark.parametrize("kind,ms", [("actorder", (300, 1)), ("actorder", (16, 2)), ("padded", (256, 3))])
def test_noalloc_matches_workspace_entry_point(kind, ms):
    from onecomp_runtime import _hip, synthetic

    mod = _layer(kind)
    for M in ms:  # the second call has the smaller input
        x = synthetic.activations(M, mod.in_features, seed=20610 + M).to(DEV)
        ref = torch.empty((M, mod.out_features), dtype=x.dtype, device=DEV)
        got = torch.full_like(ref, float("nan"))
        ws = _hip.gemm_workspace(0, M, mod.out_features, mod.k_phys, mod.group_rows, mod.kmap is not None, 0)
        say(f"noalloc {kind} M={M}: workspace entry point")
        assert _call("oc_int4_gemm", mod, x, ref, ws) == 0
        say(f"noalloc {kind} M={M}: allocation-free entry point")
        assert _call("oc_int4_gemm_noalloc", mod, x, got) == 0, _hip.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"{kind} M={M}"


def test_noalloc_rejects_calls_beyond_the_scratch():
    from onecomp_runtime import _hip, synthetic

    cap = _hip.lib().oc_int4_gemm_noalloc_scratch_bytes()
    assert cap == 32 << 20
    mod = _layer("actorder")
    M = 4096  # gathered activations alone: 4096 x 5120 x 2 B = 40 MiB
    need = _hip.gemm_workspace_bytes(M, mod.out_features, mod.k_phys, mod.group_rows, True, 0)
    assert need > cap
    x = synthetic.activations(M, mod.in_features, seed=20620).to(DEV)
    out = torch.empty((M, mod.out_features), dtype=x.dtype, device=DEV)
    say("noalloc over the scratch limit (host-side rejection)")
    status = _call("oc_int4_gemm_noalloc", mod, x, out)
    assert status == _hip.OC_ERR_WORKSPACE and "static scratch" in _hip.last_error()
