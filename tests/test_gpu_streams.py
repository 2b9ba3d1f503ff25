"""Calls on different HIP streams that overlap in time use separate GEMM
workspaces: a decode layer whose balanced ranges cut tiles (partials swapped
through the workspace's counter cells) and a split-K act-order layer (fp32
partials, and activation rows gathered into the workspace: K beyond what the
tiled kernel gathers in its loads) run concurrently, many times, on two
streams; every output equals the single-stream result bit for bit and
matches the oracle."""
import pytest
import torch

from gpu_helpers import assert_gemm_close, layer_oracle_inputs, np32, say
from oracle import onecomp_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_two_streams_overlapping_calls():
    from onecomp_runtime import kernels, synthetic
    from onecomp_runtime.layers import PackedGPTQLinear

    dec = synthetic.gptq_layer(5120, 17408, seed=20500, act_order=True)
    sk = synthetic.gptq_layer(9216, 2048, seed=20501, act_order=True)
    a = PackedGPTQLinear(5120, 17408, dec.qweight.to(DEV), dec.scales.to(DEV), dec.qzeros.to(DEV),
                         g_idx=dec.g_idx.to(DEV), groupsize=32)
    b = PackedGPTQLinear(9216, 2048, sk.qweight.to(DEV), sk.scales.to(DEV), sk.qzeros.to(DEV),
                         g_idx=sk.g_idx.to(DEV), groupsize=32)
    xa = synthetic.activations(1, 5120, seed=20502).to(DEV)
    xb = synthetic.activations(96, 9216, seed=20503).to(DEV)
    # the decode call uses the counter cells, the act-order one gathered rows and split-K partials
    from onecomp_runtime import _hip

    assert _hip.gemm_workspace_bytes(1, 17408, a.k_phys, a.group_rows, True, 0) > 0
    assert _hip.gemm_workspace_bytes(96, 2048, b.k_phys, b.group_rows, True, 0) > 512 * 1024 + 96 * 9216 * 2
    say("two streams: single-stream references")
    with torch.no_grad():
        ref_a, ref_b = a(xa), b(xb)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs_a, outs_b = [], []
    say("two streams: 40 interleaved rounds")
    with torch.no_grad():
        for _ in range(40):
            with torch.cuda.stream(s1):
                outs_a.append(a(xa))
            with torch.cuda.stream(s2):
                outs_b.append(b(xb))
                outs_b.append(b(xb))
    torch.cuda.synchronize()
    assert all(torch.equal(o, ref_a) for o in outs_a)
    assert all(torch.equal(o, ref_b) for o in outs_b)
    keys = {k for k in _hip.workspace._bufs if k[0] == 0}
    assert {(0, s1.cuda_stream), (0, s2.cuda_stream)} <= keys
    assert_gemm_close(ref_a, O.gptq_linear(np32(xa), *layer_oracle_inputs(dec), 5120, 17408, "bf16"), "decode")
    assert_gemm_close(ref_b, O.gptq_linear(np32(xb), *layer_oracle_inputs(sk), 9216, 2048, "bf16"), "split-K act-order")
