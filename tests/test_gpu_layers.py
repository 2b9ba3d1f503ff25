"""RTN linear / embedding, the MoE grouped GEMM, and the reference-API
surface (backend builders, functional GEMM, loader) on the GPU."""
import json

import numpy as np
import pytest
import torch

from gpu_helpers import assert_gemm_close, bits16, layer_oracle_inputs, np32, oracle_bits, say
from oracle import onecomp_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


# -- RTN ------------------------------------------------------------------------
def test_rtn_linear_workload():
    from onecomp_runtime import PackedRTNLinear, synthetic

    say("rtn linear M=512 K=1024 N=2048")
    layer = synthetic.rtn_layer(2048, 1024, seed=20300)
    x = synthetic.activations(512, 1024, seed=20301)
    mod = PackedRTNLinear(1024, 2048, layer.qweight_u8.to(DEV), layer.scales.to(DEV), layer.zeros.to(DEV))
    ref = O.rtn_linear(np32(x), layer.qweight_u8.numpy(), layer.scales.float().numpy(),
                       layer.zeros.float().numpy(), 1024, 2048, "bf16")
    assert_gemm_close(mod(x.to(DEV)), ref, "rtn linear")


@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 64, 65, 200])
@pytest.mark.parametrize("G", [1, 4])
def test_rtn_linear_one_hot_bit_exact(M, G):
    """The fused RTN kernels' per-op-rounded dequant is bit-exact (M <= 4: the
    row GEMV, one wave per output row; larger M: the tiled kernel)."""
    from onecomp_runtime import PackedRTNLinear

    rng = np.random.default_rng(M + G)
    K, N = 256, 96
    q = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((N, G))) * 0.05 + 1e-3).astype(np.float16)
    z = rng.uniform(-3, 18, (N, G)).astype(np.float16)
    mod = PackedRTNLinear(K, N, torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV),
                          torch.from_numpy(z).to(DEV))
    wd = O.rtn_dequant(q, s.astype(np.float32), z.astype(np.float32), K, N, "bf16")
    ks = rng.integers(0, K, M)
    x = torch.zeros((M, K), dtype=torch.bfloat16)
    x[torch.arange(M), torch.from_numpy(ks)] = 1.0
    say(f"rtn one-hot M={M} G={G}")
    out = mod(x.to(DEV))
    assert np.array_equal(bits16(out), oracle_bits(wd[:, ks].T, torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [7, 200])
def test_rtn_linear_exact_shortcut_and_general_groups(dtype, M):
    """Integral zeros (|z| <= 240) with positive scales take the kernel's
    single-rounding shortcut; fractional or large zeros and zero or negative
    scales the per-op path. Both within one layer (mixed per wave and per
    step), one-hot inputs: bit-exact against the per-op-rounded oracle
    (+ 0.0: a GEMM output carries no negative zero)."""
    from onecomp_runtime import PackedRTNLinear

    rng = np.random.default_rng(31 + M)
    K, N, G = 256, 96, 4
    q = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((N, G))) * 0.05 + 1e-3).astype(np.float16)
    z = rng.integers(0, 16, (N, G)).astype(np.float16)
    z[0:16, 1] = 240.0        # shortcut bound
    z[16:32, 2] = -240.0
    z[32, 0] = 241.0          # past the bound: per-op path for that wave's step
    z[40, 3] = 7.5            # fractional
    z[48:64, :] = 300.0       # large: RNE(c - z) rounds in bf16
    s[64, 1] = -0.02          # negative scale
    s[80, 2] = 0.0            # zero scale
    mod = PackedRTNLinear(K, N, torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV),
                          torch.from_numpy(z).to(DEV))
    fmt = "bf16" if dtype == torch.bfloat16 else "f16"
    wd = O.rtn_dequant(q, s.astype(np.float32), z.astype(np.float32), K, N, fmt)
    ks = rng.integers(0, K, M)
    x = torch.zeros((M, K), dtype=dtype)
    x[torch.arange(M), torch.from_numpy(ks)] = 1.0
    say(f"rtn shortcut/general mix M={M} {dtype}")
    assert np.array_equal(bits16(mod(x.to(DEV))), oracle_bits(wd[:, ks].T + 0.0, dtype))


@pytest.mark.parametrize("N", [24, 40])
@pytest.mark.parametrize("M", [1, 65, 200])
def test_rtn_linear_ragged_tile_n(N, M):
    """N % 16 == 8: the last 16-column tile is half full (its upper lanes'
    weight rows are clamped, never read past the table)."""
    from onecomp_runtime import PackedRTNLinear

    rng = np.random.default_rng(N * 1000 + M)
    K, G = 256, 2
    q = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((N, G))) * 0.05 + 1e-3).astype(np.float16)
    z = rng.integers(0, 16, (N, G)).astype(np.float16)
    mod = PackedRTNLinear(K, N, torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV),
                          torch.from_numpy(z).to(DEV))
    assert mod._fused_ok(torch.zeros(1, K, dtype=torch.bfloat16))
    wd = O.rtn_dequant(q, s.astype(np.float32), z.astype(np.float32), K, N, "bf16")
    ks = rng.integers(0, K, M)
    x = torch.zeros((M, K), dtype=torch.bfloat16)
    x[torch.arange(M), torch.from_numpy(ks)] = 1.0
    say(f"rtn ragged tile N={N} M={M} one-hot")
    assert np.array_equal(bits16(mod(x.to(DEV))), oracle_bits(wd[:, ks].T, torch.bfloat16))
    xr = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    say(f"rtn ragged tile N={N} M={M} random")
    ref = O.rtn_linear(np32(xr), q, s.astype(np.float32), z.astype(np.float32), K, N, "bf16")
    assert_gemm_close(mod(xr.to(DEV)), ref, f"rtn N={N} M={M}")


def test_rtn_linear_bias_and_fp32_path():
    from onecomp_runtime import PackedRTNLinear, synthetic

    layer = synthetic.rtn_layer(64, 96, seed=5)  # K % 32 == 0, G = 1
    bias = torch.randn(64, generator=torch.Generator().manual_seed(2))
    mod = PackedRTNLinear(96, 64, layer.qweight_u8.to(DEV), layer.scales.to(DEV), layer.zeros.to(DEV),
                          bias=bias.to(DEV))
    x = synthetic.activations(10, 96, seed=6)
    args = (layer.qweight_u8.numpy(), layer.scales.float().numpy(), layer.zeros.float().numpy(), 96, 64)
    say("rtn bias bf16")
    assert_gemm_close(mod(x.to(DEV)), O.rtn_linear(np32(x), *args, "bf16", bias=bias.numpy()), "rtn bias")
    say("rtn fp32 path")
    out = mod(x.float().to(DEV))
    assert out.dtype == torch.float32
    assert_gemm_close(out, O.rtn_linear(np32(x), *args, "f32", bias=bias.numpy()), "rtn fp32")
    odd = synthetic.rtn_layer(16, 10, seed=7)  # K = 10: not fused, dequant + F.linear on device
    mod2 = PackedRTNLinear(10, 16, odd.qweight_u8.to(DEV), odd.scales.to(DEV), odd.zeros.to(DEV))
    x2 = synthetic.activations(3, 10, seed=8)
    say("rtn odd K")
    assert_gemm_close(mod2(x2.to(DEV)), O.rtn_linear(np32(x2), odd.qweight_u8.numpy(),
                                                      odd.scales.float().numpy(),
                                                      odd.zeros.float().numpy(), 10, 16, "bf16"), "odd K")


@pytest.mark.parametrize("G", [1, 32])
@pytest.mark.parametrize("scale_dtype,zero_dtype", [(torch.float16, torch.float16),
                                                    (torch.bfloat16, torch.float16),
                                                    (torch.bfloat16, torch.bfloat16)])
def test_embedding_workload_bit_exact(G, scale_dtype, zero_dtype):
    from onecomp_runtime import PackedEmbedding, synthetic

    V, D, T = 32768, 1024, 4096
    layer = synthetic.rtn_layer(V, D, seed=20310, groups=G)
    scales, zeros = layer.scales.to(scale_dtype), layer.zeros.to(zero_dtype)
    ids = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(20311))
    emb = PackedEmbedding(V, D, layer.qweight_u8.to(DEV), scales.to(DEV), zeros.to(DEV))
    say(f"embedding G={G} scales={scale_dtype} zeros={zero_dtype}")
    out = emb(ids.to(DEV))
    assert out.dtype == scale_dtype and out.shape == (T, D)
    fmt = "bf16" if scale_dtype == torch.bfloat16 else "f16"
    ref = O.embedding(ids.numpy(), layer.qweight_u8.numpy(), scales.float().numpy(),
                      zeros.float().numpy(), D, fmt)
    assert np.array_equal(bits16(out), oracle_bits(ref, scale_dtype))


def test_embedding_shapes_negative_and_bad_ids():
    from onecomp_runtime import PackedEmbedding, synthetic

    V, D = 100, 20  # D % 16 != 0: scalar path
    layer = synthetic.rtn_layer(V, D, seed=9)
    emb = PackedEmbedding(V, D, layer.qweight_u8.to(DEV), layer.scales.to(DEV), layer.zeros.to(DEV))
    ids = torch.tensor([[1, -1, 99], [0, 5, 5]])
    say("embedding 2-D ids with a negative id")
    out = emb(ids.to(DEV))
    assert out.shape == (2, 3, D)
    ref = O.embedding(ids.numpy(), layer.qweight_u8.numpy(), layer.scales.float().numpy(),
                      layer.zeros.float().numpy(), D, "f16")
    assert np.array_equal(bits16(out.reshape(6, D)), oracle_bits(ref, torch.float16))
    emb.check_ids()
    say("embedding out-of-range id")
    out = emb(torch.tensor([3, V], device=DEV))
    assert torch.all(out[1] == 0)
    with pytest.raises(IndexError):
        emb.check_ids()
    emb.check_ids()  # flag cleared


# -- MoE ------------------------------------------------------------------------
def test_moe_route_matches_stable_sort():
    from onecomp_runtime import kernels, synthetic

    T, E, topk = 512, 64, 8
    ids = synthetic.router_topk(T, E, topk, seed=20320)
    say("moe route")
    off, pairs = kernels.moe_route(ids.to(DEV), E)
    flat = ids.reshape(-1).numpy()
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)
    assert np.array_equal(off.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    assert np.array_equal(pairs.cpu().numpy(), order)


def test_moe_route_drops_invalid_ids():
    from onecomp_runtime import kernels

    ids = torch.tensor([[0, 3], [7, -1], [3, 3]])
    say("moe route invalid ids")
    off, pairs = kernels.moe_route(ids.to(DEV), 4)
    assert off.cpu().tolist() == [0, 1, 1, 1, 4]
    assert pairs.cpu().tolist()[:4] == [0, 1, 4, 5]


@pytest.mark.parametrize("T,topk,E,kind", [(512, 8, 64, "skewed"), (8192, 8, 1024, "uniform"),
                                            (300, 3, 100, "invalid"), (77, 1, 1, "uniform"),
                                            (1000, 5, 33, "invalid")])
def test_moe_route_stable_sort_shapes(T, topk, E, kind):
    """Ranks of same-expert pairs within 64-pair batches, per-wave counters
    and the expert scan give numpy's stable order; ids outside [0, E) drop."""
    from onecomp_runtime import kernels

    rng = np.random.default_rng(T + E)
    if kind == "skewed":  # most pairs on two experts
        flat = np.where(rng.random(T * topk) < 0.9, rng.integers(0, 2, T * topk), rng.integers(0, E, T * topk))
    else:
        flat = rng.integers(0, E, T * topk)
    if kind == "invalid":
        bad = rng.random(T * topk) < 0.2
        flat = np.where(bad, rng.choice([-1, E, E + 5], T * topk), flat)
    ids = torch.from_numpy(flat.reshape(T, topk).astype(np.int64))
    say(f"moe route T={T} topk={topk} E={E} {kind}")
    off, pairs = kernels.moe_route(ids.to(DEV), E)
    valid = (flat >= 0) & (flat < E)
    order = np.argsort(np.where(valid, flat, E), kind="stable")[: int(valid.sum())]
    counts = np.bincount(flat[valid], minlength=E)
    assert np.array_equal(off.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    assert np.array_equal(pairs.cpu().numpy()[: int(valid.sum())], order)


@pytest.mark.parametrize("E,K,N,T,topk", [(64, 4096, 2048, 512, 8), (8, 512, 256, 37, 2)])
def test_moe_grouped_gemm(E, K, N, T, topk):
    from onecomp_runtime import kernels, synthetic

    say(f"moe grouped gemm E={E} K={K} N={N} T={T} topk={topk}")
    experts = synthetic.moe_experts(E, K, N, seed=20330)
    x = synthetic.activations(T, K, seed=20331)
    ids = synthetic.router_topk(T, E, topk, seed=20332)
    off, pairs = kernels.moe_route(ids.to(DEV), E)
    w = kernels.prepare_experts(experts.qweight.to(DEV), experts.scales.to(DEV), experts.qzeros.to(DEV))
    y = kernels.int4_moe_gemm(x.to(DEV), topk, w, off, pairs)
    assert y.shape == (T * topk, N)
    used = np.unique(ids.numpy())
    ws = {}
    for e in used:
        qw, sc, qz, g = layer_oracle_inputs(experts.layers[e])
        ws[int(e)] = O.dequant_gptq(qw, sc, qz, g, K, N, "bf16")
    ref = O.moe(np32(x), ids.numpy(), ws, "bf16")
    assert_gemm_close(y, ref, "moe")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_moe_grouped_gemm_one_hot_bit_exact(dtype):
    """In-kernel dequant of the grouped GEMM, bit for bit: token t's row is
    e_{k_t}, so Y[t*topk + j] = Wd_{e(t,j)}[:, k_t]. Skewed routing: expert 0
    takes every token (300 rows: three 128-row blocks, the last partial),
    experts 1-3 share the second slot, experts 4-7 get no rows."""
    from onecomp_runtime import kernels, synthetic

    E, K, N, T, topk = 8, 512, 192, 300, 2
    experts = synthetic.moe_experts(E, K, N, seed=20340)
    ids = torch.stack([torch.zeros(T, dtype=torch.int64), 1 + torch.arange(T) % 3], dim=1)
    rng = np.random.default_rng(20341)
    ks = rng.integers(0, K, T)
    x = torch.zeros((T, K), dtype=dtype)
    x[torch.arange(T), torch.from_numpy(ks)] = 1.0
    say(f"moe one-hot E={E} T={T} {dtype}")
    off, pairs = kernels.moe_route(ids.to(DEV), E)
    assert off.cpu().tolist() == [0, 300, 400, 500, 600, 600, 600, 600, 600]
    w = kernels.prepare_experts(experts.qweight.to(DEV), experts.scales.to(DEV), experts.qzeros.to(DEV))
    y = kernels.int4_moe_gemm(x.to(DEV), topk, w, off, pairs)
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    wds = {e: O.dequant_gptq(*layer_oracle_inputs(experts.layers[e]), K, N, name) for e in range(4)}
    expect = np.stack([wds[int(ids[t, j])][:, ks[t]] for t in range(T) for j in range(topk)])
    assert np.array_equal(bits16(y), oracle_bits(expect, dtype))


# -- reference API surface -----------------------------------------------------
def test_functional_fused_int4_gemm():
    from onecomp_runtime import fused_int4_gemm, synthetic

    layer = synthetic.gptq_layer(512, 256, seed=70)
    x = synthetic.activations(6, 512, seed=71)
    say("fused_int4_gemm functional")
    out = fused_int4_gemm(x.to(DEV), layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV))
    # the functional path casts scales to the activation dtype (bf16) first
    qw, sc, qz, g = layer_oracle_inputs(layer)
    sc_bf16 = O.round_to(sc, "bf16")
    ref = O.gptq_linear(np32(x), qw, sc_bf16, qz, g, 512, 256, "bf16")
    assert_gemm_close(out, ref, "functional")
    with pytest.raises(AssertionError):
        fused_int4_gemm(x.to(DEV), layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                        groupsize=64)


@pytest.mark.parametrize("backend_name,kind", [("hip", "hip"), ("fused", "fused"), ("packed", "packed"),
                                               ("eager", "eager")])
@pytest.mark.parametrize("case", ["gs32", "actorder", "gs26", "gs128", "v2"])
def test_build_quant_layer_routes(backend_name, kind, case):
    from onecomp_runtime import backend, synthetic

    K, N, gs = 512, 128, 32
    kw = {}
    if case == "gs26":
        K, gs = 520, 26
    if case == "gs128":
        gs = 128
    if case == "actorder":
        kw["act_order"] = True
    if case == "v2":
        kw["v1"] = False
    layer = synthetic.gptq_layer(K, N, seed=80, groupsize=gs, **kw)
    entry = dict(in_features=K, out_features=N, wbits=4, groupsize=gs, actorder=layer.g_idx is not None,
                 checkpoint_format="gptq" if layer.v1 else "gptq_v2", name="blk.proj")
    st = dict(qweight=layer.qweight, scales=layer.scales, qzeros=layer.qzeros)
    if layer.g_idx is not None:
        st["g_idx"] = layer.g_idx
    say(f"build_quant_layer backend={backend_name} case={case}")
    mod, got_kind = backend.build_quant_layer(entry, st, backend_name, torch.bfloat16, torch.device(DEV))
    if backend_name == "fused" and case == "actorder":
        assert got_kind == "packed"
    else:
        assert got_kind == kind
    x = synthetic.activations(5, K, seed=81)
    qw, sc, qz, g = layer_oracle_inputs(layer)
    if backend_name == "packed":
        sc = O.round_to(sc, "bf16")  # build_packed casts scales to the compute dtype
    ref = O.gptq_linear(np32(x), qw, sc, qz, g, K, N, "bf16", layer.v1)
    assert_gemm_close(mod(x.to(DEV)), ref, f"{backend_name}/{case}")


def test_packed_gptq_8bit_and_fp32():
    from onecomp_runtime import PackedGPTQLinear

    rng = np.random.default_rng(90)
    K, N, gs = 256, 64, 64
    codes = rng.integers(0, 256, (K, N))
    zeros = rng.integers(0, 256, (K // gs, N))
    scales = (np.abs(rng.standard_normal((K // gs, N))) * 0.001 + 1e-4).astype(np.float16)
    qw, qz = O.pack_rows(codes, 8), O.pack_zeros(zeros, True, 8)
    mod = PackedGPTQLinear(K, N, torch.from_numpy(qw).to(DEV), torch.from_numpy(scales).to(DEV),
                           torch.from_numpy(qz).to(DEV), groupsize=gs, wbits=8)
    x = torch.randn(4, K, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    say("packed 8-bit")
    ref = O.gptq_linear(np32(x), qw, scales.astype(np.float32), qz, O.default_g_idx(K, gs), K, N, "bf16",
                        wbits=8)
    assert_gemm_close(mod(x.to(DEV)), ref, "8-bit")
    say("packed fp32 activations")
    from onecomp_runtime import synthetic

    layer = synthetic.gptq_layer(256, 64, seed=91, act_order=True)
    m4 = PackedGPTQLinear(256, 64, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                          g_idx=layer.g_idx.to(DEV), groupsize=32)
    xf = torch.randn(3, 256, generator=torch.Generator().manual_seed(4))
    out = m4(xf.to(DEV))
    assert out.dtype == torch.float32
    a, b, c, g = layer_oracle_inputs(layer)
    assert_gemm_close(out, O.gptq_linear(xf.numpy(), a, b, c, g, 256, 64, "f32"), "fp32 packed")


@pytest.mark.parametrize("M", [1, 6, 100])
def test_packed_gptq_bias_rounded_to_activation_dtype(M):
    """PackedGPTQLinear adds ``bias.to(x.dtype)`` (packed_gptq_linear.py:73):
    with one-hot rows the output is RNE(Wd[:, k] + RNE_bf16(bias)) exactly.
    FusedInt4Linear adds the stored bias as is (the reference's kernels do)."""
    from onecomp_runtime import FusedInt4Linear, PackedGPTQLinear, synthetic

    K, N = 512, 64
    # Power-of-two scales: every s * (w - z) is exact in bf16, so the decode
    # kernel's unrounded products and the dequantize-then-multiply order agree
    # and the comparison isolates the bias rounding.
    gen = torch.Generator().manual_seed(8)

    def pow2_scales(layer):
        layer.scales = torch.pow(2.0, -torch.randint(2, 9, layer.scales.shape, generator=gen).float()).half()
        return layer

    layer = pow2_scales(synthetic.gptq_layer(K, N, seed=96, act_order=True))
    bias = torch.randn(N, generator=torch.Generator().manual_seed(7)) * 3.0  # fp32
    mod = PackedGPTQLinear(K, N, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                           g_idx=layer.g_idx.to(DEV), bias=bias.to(DEV), groupsize=32)
    rng = np.random.default_rng(M)
    ks = rng.integers(0, K, M)
    x = torch.zeros((M, K), dtype=torch.bfloat16)
    x[torch.arange(M), torch.from_numpy(ks)] = 1.0
    wd = O.dequant_gptq(*layer_oracle_inputs(layer), K, N, "bf16")
    say(f"packed fp32 bias M={M}")
    expect = O.round_to(wd[:, ks].T + O.round_to(bias.numpy(), "bf16")[None, :], "bf16")
    assert np.array_equal(bits16(mod(x.to(DEV))), oracle_bits(expect, torch.bfloat16))
    plain = pow2_scales(synthetic.gptq_layer(K, N, seed=97))
    fmod = FusedInt4Linear(K, N, plain.qweight.to(DEV), plain.scales.to(DEV), plain.qzeros.to(DEV),
                           bias=bias.to(DEV))
    wd2 = O.dequant_gptq(*layer_oracle_inputs(plain), K, N, "bf16")
    expect2 = O.round_to(wd2[:, ks].T + bias.numpy()[None, :], "bf16")
    assert np.array_equal(bits16(fmod(x.to(DEV))), oracle_bits(expect2, torch.bfloat16))


def test_module_dtype_moves_keep_packed_buffers():
    from onecomp_runtime import synthetic
    from onecomp_runtime.layers import FusedInt4LinearPaddedGroups

    layer = synthetic.gptq_layer(104, 64, seed=92, groupsize=26)
    mod = FusedInt4LinearPaddedGroups(104, 64, layer.qweight.to(DEV), layer.scales.to(DEV),
                                      layer.qzeros.to(DEV), groupsize=26)
    say("module .to(dtype)")
    mod = mod.to(torch.float32)
    assert mod.qweight_tiled.dtype == torch.int32 and mod.zeros_tiled.dtype == torch.int32
    assert mod.kmap.dtype == torch.int32 and mod.scales_tiled.dtype == torch.float16
    mod.warmup((1, 40))
    x = synthetic.activations(3, 104, seed=93)
    assert_gemm_close(mod(x.to(DEV)), O.gptq_linear(np32(x), *layer_oracle_inputs(layer), 104, 64, "bf16"),
                      "after .to")


def test_layer_built_on_host_prepares_on_first_device_forward():
    """A layer constructed from CPU tensors (the reference allows it) keeps the
    checkpoint tensors until it is moved; the first device forward tiles them."""
    from onecomp_runtime import synthetic
    from onecomp_runtime.layers import PackedGPTQLinear

    layer = synthetic.gptq_layer(512, 96, seed=94, act_order=True, v1=False)
    mod = PackedGPTQLinear(512, 96, layer.qweight, layer.scales, layer.qzeros, g_idx=layer.g_idx,
                           groupsize=32, v1=False)
    assert mod.qweight_tiled is None
    with pytest.raises(RuntimeError):
        mod.tiled()
    mod = mod.to(DEV)
    x = synthetic.activations(5, 512, seed=95)
    say("host-built layer, first device forward")
    out = mod(x.to(DEV))
    assert mod.qweight_tiled is not None and mod._src_qweight is None
    assert_gemm_close(out, O.gptq_linear(np32(x), *layer_oracle_inputs(layer), 512, 96, "bf16", False),
                      "host-built")
    wd = O.dequant_gptq(*layer_oracle_inputs(layer), 512, 96, "f16", False)
    assert np.array_equal(bits16(mod.dequantize(torch.float16)), oracle_bits(wd, torch.float16))


class _TinyBlock(torch.nn.Module):
    def __init__(self, cfg):
        super().__init__()
        d, h = cfg["dim"], cfg["hidden"]
        self.norm = torch.nn.LayerNorm(d)
        self.up = torch.nn.Linear(d, h)
        self.down = torch.nn.Linear(h, d, bias=False)

    def forward(self, x):
        return self.down(torch.nn.functional.gelu(self.up(self.norm(x))))


def test_load_int4_model_end_to_end(tmp_path):
    from safetensors.torch import save_file

    from onecomp_runtime import load_int4_model, synthetic

    d, h = 256, 512
    up = synthetic.gptq_layer(d, h, seed=100)
    down = synthetic.gptq_layer(h, d, seed=101, act_order=True, v1=False)
    bias = torch.randn(h, generator=torch.Generator().manual_seed(5)).to(torch.float16)
    tensors = {
        "norm.weight": torch.ones(d), "norm.bias": torch.zeros(d),
        "up.qweight": up.qweight, "up.scales": up.scales, "up.qzeros": up.qzeros, "up.bias": bias,
        "down.qweight": down.qweight, "down.scales": down.scales, "down.qzeros": down.qzeros,
        "down.g_idx": down.g_idx.to(torch.int32),
    }
    layers = [dict(name="up", wbits=4, groupsize=32, actorder=False, in_features=d, out_features=h),
              dict(name="down", wbits=4, groupsize=32, actorder=True, in_features=h, out_features=d)]
    path = tmp_path / "tiny.safetensors"
    save_file(tensors, str(path), metadata={"config_json": json.dumps({"dim": d, "hidden": h}),
                                            "quant_layers_json": json.dumps(layers),
                                            "checkpoint_format": "gptq_v2"})
    say("load_int4_model end to end")
    model = load_int4_model(str(path), _TinyBlock, device=DEV, dtype="bfloat16", backend="auto",
                            warmup_m_values=(1, 64))
    assert type(model.up).__name__ == "FusedInt4Linear" and not model.up.v1
    assert type(model.down).__name__ == "PackedGPTQLinear"
    x = synthetic.activations(7, d, seed=102)
    with torch.no_grad():
        out = model(x.to(DEV))
    # oracle: same block with eager-dequantized weights (v2 zeros)
    xn = torch.nn.functional.layer_norm(x.float(), (d,)).to(torch.bfloat16)
    a1 = O.gptq_linear(np32(xn), up.qweight.numpy(), up.scales.float().numpy(), up.qzeros.numpy(),
                       O.default_g_idx(d, 32), d, h, "bf16", v1=False, bias=bias.float().numpy())
    g1 = torch.nn.functional.gelu(torch.from_numpy(a1).to(torch.bfloat16)).float().numpy()
    ref = O.gptq_linear(g1, down.qweight.numpy(), down.scales.float().numpy(), down.qzeros.numpy(),
                        down.g_idx.numpy(), h, d, "bf16", v1=False)
    assert_gemm_close(out, ref, "tiny model")
