"""Fused 8-bit GPTQ (wbits = 8: 4 codes per word, mask 0xFF; quant_utils.py:
21-22): PackedGPTQLinear(wbits=8) runs oc_int8_gemm on its tiled layout and
never materialises a dense weight. In-GEMM dequant bit-exact through one-hot
rows; outputs within the GEMM tolerance of the oracle (dequant_gptq_to_fp +
F.linear); module state read back verbatim."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_gemm_close, bits16, np32, oracle_bits, say
from oracle import onecomp_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _layer8(K, N, gs, seed, act_order=False, v1=True, scale_dtype=np.float16):
    rng = np.random.default_rng(seed)
    G = (K + gs - 1) // gs
    codes = rng.integers(0, 256, (K, N))
    zeros = rng.integers(0, 256, (G, N))
    scales = (np.abs(rng.standard_normal((G, N))) * 0.001 + 1e-4).astype(scale_dtype)
    g = (rng.permutation(K) // gs) if act_order else O.default_g_idx(K, gs)
    return dict(qw=O.pack_rows(codes, 8), qz=O.pack_zeros(zeros, v1, 8), sc=scales, g=g, K=K, N=N, gs=gs, v1=v1,
                act=act_order)


def _module(L, dev=DEV):
    from onecomp_runtime import PackedGPTQLinear

    g = torch.from_numpy(L["g"]).to(dev) if L["act"] else None
    return PackedGPTQLinear(L["K"], L["N"], torch.from_numpy(L["qw"]).to(dev), torch.from_numpy(L["sc"]).to(dev),
                            torch.from_numpy(L["qz"]).to(dev), g_idx=g, groupsize=L["gs"], wbits=8, v1=L["v1"])


def _wd(L, dtype):
    return O.dequant_gptq(L["qw"], L["sc"].astype(np.float32), L["qz"], L["g"], L["K"], L["N"], dtype, L["v1"],
                          wbits=8)


@pytest.mark.parametrize("case", ["gs128_k5120", "actorder_v1", "v2_gs32_fp16", "ragged_k"])
@pytest.mark.parametrize("M", [1, 7, 300])
def test_int8_one_hot_bit_exact(case, M):
    K, N, gs, kw = 5120, 5120, 128, {}
    dt = torch.bfloat16
    if case == "actorder_v1":
        K, N, gs, kw = 1024, 256, 32, dict(act_order=True)
    elif case == "v2_gs32_fp16":
        K, N, gs, kw, dt = 1024, 192, 32, dict(v1=False), torch.float16
    elif case == "ragged_k":
        K, N, gs = 1000, 132, 64
    L = _layer8(K, N, gs, seed=hash(case) % 997 + M, **kw)
    mod = _module(L)
    assert type(mod.qweight_tiled) is torch.Tensor and mod.qweight_tiled.shape[-1] == 8
    rng = np.random.default_rng(M)
    ks = rng.integers(0, K, M)
    x = torch.zeros((M, K), dtype=dt)
    x[torch.arange(M), torch.from_numpy(ks)] = 1.0
    say(f"int8 one-hot {case} M={M}")
    out = mod(x.to(DEV))
    name = "bf16" if dt == torch.bfloat16 else "f16"
    assert np.array_equal(bits16(out), oracle_bits(_wd(L, name)[:, ks].T, dt))


@pytest.mark.parametrize("M", [1, 8, 64, 600])
def test_int8_gemm_matches_oracle(M):
    L = _layer8(5120, 5120, 128, seed=20400)
    mod = _module(L)
    x = torch.randn(M, 5120, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    say(f"int8 gemm M={M} K=N=5120 gs128")
    ref = O.gptq_linear(np32(x), L["qw"], L["sc"].astype(np.float32), L["qz"], L["g"], 5120, 5120, "bf16",
                        wbits=8)
    assert_gemm_close(mod(x.to(DEV)), ref, f"int8 M={M}")


def test_int8_act_order_bias_fp32_and_state():
    L = _layer8(768, 96, 32, seed=20410, act_order=True)
    from onecomp_runtime import PackedGPTQLinear

    bias = torch.randn(96, generator=torch.Generator().manual_seed(2))
    mod = PackedGPTQLinear(768, 96, torch.from_numpy(L["qw"]).to(DEV), torch.from_numpy(L["sc"]).to(DEV),
                           torch.from_numpy(L["qz"]).to(DEV), g_idx=torch.from_numpy(L["g"]).to(DEV),
                           bias=bias.to(DEV), groupsize=32, wbits=8)
    x = torch.randn(5, 768, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    say("int8 act-order with bias")
    ref = O.gptq_linear(np32(x), L["qw"], L["sc"].astype(np.float32), L["qz"], L["g"], 768, 96, "bf16",
                        bias=bias.numpy(), wbits=8)
    assert_gemm_close(mod(x.to(DEV)), ref, "int8 act-order bias")
    xf = torch.randn(3, 768, generator=torch.Generator().manual_seed(4))
    say("int8 fp32 activations")
    out = mod(xf.to(DEV))
    assert out.dtype == torch.float32
    assert_gemm_close(out, O.gptq_linear(xf.numpy(), L["qw"], L["sc"].astype(np.float32), L["qz"], L["g"], 768, 96,
                                         "f32", bias=bias.numpy(), wbits=8), "int8 fp32")
    wd = mod.dequantize(torch.bfloat16)
    assert np.array_equal(bits16(wd), oracle_bits(_wd(L, "bf16"), torch.bfloat16))
    sd = mod.state_dict()
    assert np.array_equal(sd["qweight"].cpu().numpy(), L["qw"])
    assert np.array_equal(sd["qzeros"].cpu().numpy(), L["qz"])
    assert np.array_equal(sd["scales"].cpu().numpy(), L["sc"])
    # reload other weights through load_state_dict
    L2 = _layer8(768, 96, 32, seed=20411, act_order=True)
    mod.load_state_dict(dict(qweight=torch.from_numpy(L2["qw"]), scales=torch.from_numpy(L2["sc"]),
                             qzeros=torch.from_numpy(L2["qz"]), g_idx=torch.from_numpy(L2["g"]), bias=bias))
    ref2 = O.gptq_linear(np32(x), L2["qw"], L2["sc"].astype(np.float32), L2["qz"], L2["g"], 768, 96, "bf16",
                         bias=bias.numpy(), wbits=8)
    assert_gemm_close(mod(x.to(DEV)), ref2, "int8 reloaded")
