"""Parity of the fused int4 GEMM (both regimes) with the oracle's CPU
packed/eager path, on the benchmark workloads and on edge cases.

Tolerance (GEMM outputs, floating point): max|out - ref| <= 2e-2 * max|ref|
and cosine >= 0.9999, ref = dequant (bit-exact) + fp32-accumulated linear.
The in-GEMM dequant itself is checked bit-exactly with one-hot activations:
row m of A = e_k gives C[m, :] = Wd[:, k] exactly.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_gemm_close, bits16, layer_oracle_inputs, np32, oracle_bits, say
from oracle import onecomp_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SPLITK, TILED, AUTO, DOT = 1, 2, 0, 3


def _module_for(layer, dtype=torch.bfloat16):
    """The layer the hip backend builds for this synthetic layer."""
    from onecomp_runtime import backend

    entry = dict(in_features=layer.K, out_features=layer.N, wbits=4, groupsize=layer.groupsize,
                 actorder=layer.g_idx is not None,
                 checkpoint_format="gptq" if layer.v1 else "gptq_v2", name="l")
    st = dict(qweight=layer.qweight, scales=layer.scales, qzeros=layer.qzeros)
    if layer.g_idx is not None:
        st["g_idx"] = layer.g_idx
    mod, kind = backend.build_quant_layer(entry, st, "hip", dtype, torch.device(DEV))
    assert kind == "hip"
    return mod


def _oracle_out(layer, x: torch.Tensor, dtype="bf16", bias=None):
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    return O.gptq_linear(np32(x), qw, sc, qz, g_idx, layer.K, layer.N, dtype, layer.v1,
                         bias=None if bias is None else np32(bias))


@pytest.fixture
def decode_kernel(monkeypatch):
    """use(kind) selects the small-batch kernel: "stream" (balanced weight
    range per workgroup, the default), "global" (the same ranges, 3..16 rows
    read from global memory instead of staged), "tile" (one 16-column tile
    per workgroup) or "split" (K-split work items, M <= 2)."""
    from onecomp_runtime import _hip

    def use(kind: str) -> None:
        monkeypatch.setenv("ONECOMP_HIP_GEMV_STREAM", "1" if kind in ("stream", "global") else "0")
        monkeypatch.setenv("ONECOMP_HIP_STREAM_GLOBAL", "1" if kind == "global" else "0")
        monkeypatch.setenv("ONECOMP_HIP_GEMV_SPLIT", "1" if kind == "split" else "0")
        _hip.gemm_workspace_bytes.cache_clear()  # workspace sizes follow the kernel

    yield use
    _hip.gemm_workspace_bytes.cache_clear()


def _gemm_raw(mod, x, regime):
    from onecomp_runtime import kernels

    return kernels.int4_gemm(x, mod.tiled(), in_features=mod.in_features, kmap=mod.kmap, kinv=mod.kinv,
                             bias=mod.bias, regime=regime)


# -- benchmark workloads ------------------------------------------------------
def test_gptq_gs32_m16():
    from onecomp_runtime import synthetic

    say("gptq_gs32_m16 M=16 K=N=4096")
    layer = synthetic.gptq_layer(4096, 4096, seed=20260)
    x = synthetic.activations(16, 4096, seed=20261)
    mod = _module_for(layer)
    assert type(mod).__name__ == "FusedInt4Linear"
    out = mod(x.to(DEV))
    assert out.dtype == torch.bfloat16 and out.shape == (16, 4096)
    assert_gemm_close(out, _oracle_out(layer, x), "gptq_gs32_m16")


@pytest.mark.parametrize("K,N", [(5120, 5120), (5120, 17408), (17408, 5120), (5120, 1024)])
@pytest.mark.parametrize("M", [1, 8])
def test_decode_actorder(K, N, M):
    from onecomp_runtime import synthetic

    say(f"decode_actorder M={M} K={K} N={N}")
    layer = synthetic.gptq_layer(K, N, seed=20270 + K + N, act_order=True)
    x = synthetic.activations(M, K, seed=20271 + M)
    mod = _module_for(layer)
    assert type(mod).__name__ == "PackedGPTQLinear" and mod.kmap is not None
    assert_gemm_close(mod(x.to(DEV)), _oracle_out(layer, x), f"decode M={M} K={K} N={N}")


@pytest.mark.parametrize("K,N", [(3072, 3072), (3072, 12288), (12288, 3072)])
def test_dit_large_m_v2(K, N):
    from onecomp_runtime import synthetic

    say(f"dit_large_m M=4096 K={K} N={N} (v2)")
    layer = synthetic.gptq_layer(K, N, seed=20280 + K + N, v1=False)
    x = synthetic.activations(4096, K, seed=20281, outliers=True)
    mod = _module_for(layer)
    out = mod(x.to(DEV))
    assert_gemm_close(out, _oracle_out(layer, x), f"dit K={K} N={N}")


def test_padded_gs26():
    from onecomp_runtime import synthetic

    say("padded_gs26 M=256 K=1040 N=3072")
    layer = synthetic.gptq_layer(1040, 3072, seed=20290, groupsize=26, pad_rows_to=1056)
    x = synthetic.activations(256, 1040, seed=20291)
    mod = _module_for(layer)
    assert type(mod).__name__ == "FusedInt4LinearPaddedGroups"
    assert mod.padded_in_features == 1280
    assert_gemm_close(mod(x.to(DEV)), _oracle_out(layer, x), "padded gs26")


# -- bit-exact in-GEMM dequant via one-hot activations ------------------------
@pytest.mark.parametrize("regime", [SPLITK, TILED])
@pytest.mark.parametrize("kind", ["gs32_v1", "v2", "actorder", "gs26", "gs128", "fp16"])
def test_gemm_dequant_bit_exact_one_hot(regime, kind):
    from onecomp_runtime import synthetic

    K, N = 1024, 192
    kw = dict(seed=31)
    dtype = torch.float16 if kind == "fp16" else torch.bfloat16
    if kind == "v2":
        kw["v1"] = False
    if kind == "actorder":
        kw["act_order"] = True
    if kind == "gs26":
        K, kw["groupsize"] = 1040, 26
    if kind == "gs128":
        kw["groupsize"] = 128
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer, dtype)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    wd = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16" if dtype == torch.bfloat16 else "f16", layer.v1)
    rng = np.random.default_rng(0)
    ks = rng.choice(K, 48, replace=False)
    x = torch.zeros((48, K), dtype=dtype)
    x[torch.arange(48), torch.from_numpy(ks)] = 1.0
    say(f"one-hot dequant kind={kind} regime={regime}")
    out = _gemm_raw(mod, x.to(DEV), regime)
    assert np.array_equal(bits16(out), oracle_bits(wd[:, ks].T, dtype))


@pytest.mark.parametrize("M,K,N,kind", [(512, 1024, 192, "gs32_v1"), (600, 2048, 400, "actorder"),
                                         (512, 1040, 96, "gs26"), (513, 4096, 64, "v2"), (600, 512, 1000, "gs128"),
                                         (256, 1024, 192, "gs32_v1"), (300, 2048, 400, "actorder")])
def test_large_m_kernel_one_hot_bit_exact(M, K, N, kind):
    """The pipelined 128 x 192 kernel (512 <= M < 1024; split K when the grid
    is small) and, below 512 rows, the tiled kernel reproduce dequantized
    columns exactly."""
    from onecomp_runtime import synthetic

    kw = dict(seed=33)
    if kind == "v2":
        kw["v1"] = False
    if kind == "actorder":
        kw["act_order"] = True
    if kind == "gs26":
        kw["groupsize"] = 26
    if kind == "gs128":
        kw["groupsize"] = 128
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    wd = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16", layer.v1)
    rng = np.random.default_rng(5)
    ks = rng.integers(0, K, M)
    x = torch.zeros((M, K), dtype=torch.bfloat16)
    x[torch.arange(M), torch.from_numpy(ks)] = 1.0
    say(f"large-M one-hot M={M} K={K} N={N} kind={kind}")
    out = _gemm_raw(mod, x.to(DEV), TILED)
    assert np.array_equal(bits16(out), oracle_bits(wd[:, ks].T, torch.bfloat16))


@pytest.mark.parametrize("M,K,N,kind", [(1100, 1024, 200, "gs32_v1"), (1024, 2048, 400, "actorder"),
                                         (1030, 1040, 96, "gs26"), (1500, 512, 1000, "gs128"),
                                         (1024, 1024, 320, "fp16"), (1024, 512, 264, "bf16_scales"),
                                         (4096, 256, 12288, "v2")])
def test_wide_kernel_one_hot_bit_exact(M, K, N, kind):
    """The 256-row wave-tile kernel (M >= 1024: 192- or 256-column blocks,
    ragged M and N, gathered act-order rows, padded and wide groups, fp16
    activations, bf16 scales) reproduces dequantized columns exactly."""
    from onecomp_runtime import synthetic

    kw = dict(seed=34)
    dtype = torch.bfloat16
    if kind == "v2":
        kw["v1"] = False
    if kind == "actorder":
        kw["act_order"] = True
    if kind == "gs26":
        kw["groupsize"] = 26
    if kind == "gs128":
        kw["groupsize"] = 128
    if kind == "fp16":
        dtype = torch.float16
    if kind == "bf16_scales":
        kw["scale_dtype"] = torch.bfloat16
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer, dtype)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    wd = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16" if dtype == torch.bfloat16 else "f16", layer.v1)
    rng = np.random.default_rng(6)
    ks = rng.integers(0, K, M)
    x = torch.zeros((M, K), dtype=dtype)
    x[torch.arange(M), torch.from_numpy(ks)] = 1.0
    say(f"wide one-hot M={M} K={K} N={N} kind={kind}")
    out = _gemm_raw(mod, x.to(DEV), TILED)
    assert np.array_equal(bits16(out), oracle_bits(wd[:, ks].T, dtype))


# -- regimes and shapes -------------------------------------------------------
@pytest.mark.parametrize("M", [1, 3, 16, 17, 33, 64])
def test_splitk_and_tiled_agree_with_oracle(M):
    from onecomp_runtime import synthetic

    K, N = 2048, 640
    layer = synthetic.gptq_layer(K, N, seed=40 + M)
    x = synthetic.activations(M, K, seed=41)
    mod = _module_for(layer)
    ref = _oracle_out(layer, x)
    for regime in (SPLITK, TILED):
        say(f"regime={regime} M={M}")
        assert_gemm_close(_gemm_raw(mod, x.to(DEV), regime), ref, f"regime {regime} M={M}")


@pytest.mark.parametrize("M,K,N", [(65, 256, 8), (100, 1000, 24), (257, 512, 200), (300, 96, 64),
                                   (1, 32, 8), (2, 4096, 136)])
def test_ragged_shapes(M, K, N):
    from onecomp_runtime import synthetic

    say(f"ragged M={M} K={K} N={N}")
    layer = synthetic.gptq_layer(K, N, seed=50)
    x = synthetic.activations(M, K, seed=51)
    mod = _module_for(layer)
    assert_gemm_close(mod(x.to(DEV)), _oracle_out(layer, x), f"ragged {M}x{K}x{N}")


def test_empty_batch():
    from onecomp_runtime import synthetic

    layer = synthetic.gptq_layer(256, 64, seed=52)
    mod = _module_for(layer)
    say("empty batch")
    out = mod(torch.zeros((0, 256), dtype=torch.bfloat16, device=DEV))
    assert out.shape == (0, 64)
    out3 = mod(torch.zeros((2, 0, 256), dtype=torch.bfloat16, device=DEV))
    assert out3.shape == (2, 0, 64)


@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M", [4, 300])
def test_bias(bias_dtype, M):
    from onecomp_runtime import synthetic
    from onecomp_runtime.layers import FusedInt4Linear

    K, N = 512, 256
    layer = synthetic.gptq_layer(K, N, seed=53)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(1)).to(bias_dtype)
    mod = FusedInt4Linear(K, N, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                          bias=bias.to(DEV))
    x = synthetic.activations(M, K, seed=54)
    say(f"bias {bias_dtype} M={M}")
    ref = _oracle_out(layer, x, bias=bias.float())
    assert_gemm_close(mod(x.to(DEV)), ref, "bias")


def test_fp16_and_fp32_activations():
    from onecomp_runtime import synthetic
    from onecomp_runtime.layers import FusedInt4Linear

    K, N = 1024, 512
    layer = synthetic.gptq_layer(K, N, seed=55)
    mod = FusedInt4Linear(K, N, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV))
    x = synthetic.activations(24, K, seed=56, dtype=torch.float16)
    say("fp16 activations")
    assert_gemm_close(mod(x.to(DEV)), _oracle_out(layer, x, "f16"), "fp16")
    say("fp32 activations")
    out32 = mod(x.float().to(DEV))
    assert out32.dtype == torch.float32  # computed in fp16, returned as fp32
    assert_gemm_close(out32, _oracle_out(layer, x, "f16"), "fp32")


def test_3d_and_noncontiguous_input():
    from onecomp_runtime import synthetic

    K, N = 512, 128
    layer = synthetic.gptq_layer(K, N, seed=57)
    mod = _module_for(layer)
    x = synthetic.activations(2 * 5, K, seed=58)
    say("3-D input")
    out = mod(x.reshape(2, 5, K).to(DEV))
    assert out.shape == (2, 5, N)
    assert_gemm_close(out.reshape(10, N), _oracle_out(layer, x), "3d")
    wide = torch.zeros((10, 2 * K), dtype=torch.bfloat16)
    wide[:, ::2] = x
    say("strided input")
    assert_gemm_close(mod(wide.to(DEV)[:, ::2]), _oracle_out(layer, x), "strided")


@pytest.mark.parametrize("regime,M", [(DOT, 1), (DOT, 2), (SPLITK, 8), (TILED, 128), (TILED, 300)])
def test_deterministic(regime, M):
    """Fixed reduction orders (wave tree, split-K partials in split order)."""
    from onecomp_runtime import synthetic

    K, N = 8192, 1024
    layer = synthetic.gptq_layer(K, N, seed=59)
    mod = _module_for(layer)
    x = synthetic.activations(M, K, seed=60).to(DEV)
    say(f"determinism regime={regime} M={M}")
    a = _gemm_raw(mod, x, regime)
    b = _gemm_raw(mod, x, regime)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert_gemm_close(a, _oracle_out(layer, x.cpu()), "determinism")


def test_abi_rejects_bad_arguments():
    from onecomp_runtime import kernels, synthetic

    layer = synthetic.gptq_layer(256, 64, seed=61)
    qw, sc, qz = layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV)
    x = synthetic.activations(4, 256, seed=62).to(DEV)
    say("ABI argument errors")
    w = kernels.prepare(qw, sc, qz, in_features=256, out_features=64, kmap=None, k_phys=256, group_rows=32,
                        v1=True)
    with pytest.raises(ValueError):  # K_phys not a multiple of 32
        kernels.int4_gemm(x, kernels.TiledWeights(w.qt, w.st, w.zt, 64, 250, 32), in_features=256)
    with pytest.raises(ValueError):  # N not a multiple of 8
        kernels.int4_gemm(x, kernels.TiledWeights(w.qt, w.st, w.zt, 60, 256, 32), in_features=256)
    with pytest.raises(ValueError):  # the layout needs N % 8 == 0 as well
        kernels.prepare(qw[:, :60].contiguous(), sc[:, :60].contiguous(), qz, in_features=256, out_features=60,
                        kmap=None, k_phys=256, group_rows=32, v1=True)
    with pytest.raises(ValueError):  # group_rows must divide K_phys
        kernels.prepare(qw, sc, qz, in_features=256, out_features=64, kmap=None, k_phys=256, group_rows=96,
                        v1=True)
    with pytest.raises(NotImplementedError):  # split-K regime is for M <= 64
        kernels.int4_gemm(torch.zeros((65, 256), dtype=torch.bfloat16, device=DEV), w, in_features=256,
                          regime=SPLITK)
    with pytest.raises(NotImplementedError):  # decode regime is for M <= 2
        kernels.int4_gemm(x, w, in_features=256, regime=DOT)
    with pytest.raises(RuntimeError):  # host tensors are refused
        kernels.int4_gemm(x.cpu(), w, in_features=256)


@pytest.mark.parametrize("M", [1, 8, 200])
def test_graph_capture_replays_match_eager(M):
    """Captured launches (split-K counters and workspace included) replay
    correctly several times, with eager work in between."""
    from onecomp_runtime import synthetic

    K, N = 4096, 1024
    layer = synthetic.gptq_layer(K, N, seed=63, act_order=(M == 1))
    mod = _module_for(layer)
    x = synthetic.activations(M, K, seed=64).to(DEV)
    say(f"graph capture M={M}")
    with torch.no_grad():
        eager = mod(x).clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = mod(x)
        for rep in range(4):
            g.replay()
            other = mod(synthetic.activations(M, K, seed=65 + rep).to(DEV))  # eager work in between
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
            del other


@pytest.mark.parametrize("kernel", ["stream", "tile"])
@pytest.mark.parametrize("kind", ["gs32_v1", "v2", "actorder", "gs26", "gs128", "fp16", "bf16_scales"])
@pytest.mark.parametrize("M", [1, 2])
def test_decode_kernel_one_hot_bit_exact(kind, M, kernel, decode_kernel):
    """The decode (dot2, factored-scale) kernels reproduce dequantized rows exactly."""
    from onecomp_runtime import synthetic

    decode_kernel(kernel)
    K, N = 1024, 320
    kw = dict(seed=71)
    dtype = torch.float16 if kind == "fp16" else torch.bfloat16
    if kind == "v2":
        kw["v1"] = False
    if kind == "actorder":
        kw["act_order"] = True
    if kind == "gs26":
        K, kw["groupsize"] = 1040, 26
    if kind == "gs128":
        kw["groupsize"] = 128
    if kind == "bf16_scales":
        kw["scale_dtype"] = torch.bfloat16
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer, dtype)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    wd = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16" if dtype == torch.bfloat16 else "f16", layer.v1)
    rng = np.random.default_rng(1)
    for rep in range(3):
        ks = rng.choice(K, M, replace=False)
        x = torch.zeros((M, K), dtype=dtype)
        x[torch.arange(M), torch.from_numpy(ks)] = 1.0
        say(f"decode one-hot {kernel} kind={kind} M={M} rep={rep}")
        out = _gemm_raw(mod, x.to(DEV), DOT)
        assert np.array_equal(bits16(out), oracle_bits(wd[:, ks].T, dtype))


@pytest.mark.parametrize("kernel", ["stream", "tile"])
@pytest.mark.parametrize("K,N", [(32, 8), (1000, 200), (5120, 1024), (4096, 4096), (2048, 17408)])
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("act", [False, True])
def test_decode_kernel_matches_oracle(K, N, M, act, kernel, decode_kernel):
    from onecomp_runtime import synthetic

    decode_kernel(kernel)
    layer = synthetic.gptq_layer(K, N, seed=72 + K, act_order=act)
    x = synthetic.activations(M, K, seed=73)
    mod = _module_for(layer)
    say(f"decode kernel {kernel} K={K} N={N} M={M} act={act}")
    assert_gemm_close(_gemm_raw(mod, x.to(DEV), DOT), _oracle_out(layer, x), f"dot {K}x{N} M={M}")
    assert_gemm_close(mod(x.to(DEV)), _oracle_out(layer, x), "auto")


@pytest.mark.parametrize("K,N,gs,act", [(52, 16, 26, False), (1004, 200, 32, True), (1004, 72, 32, False),
                                         (12, 8, 32, False), (4100, 64, 128, True)])
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("kernel", ["stream", "tile"])
def test_decode_kernel_ragged_k(K, N, gs, act, M, kernel, decode_kernel):
    """K % 8 != 0 and padded groups: the decode staging scatters the tail rows
    one by one and leaves padding rows zero."""
    from onecomp_runtime import synthetic

    decode_kernel(kernel)
    layer = synthetic.gptq_layer(K, N, seed=76 + K, groupsize=gs, act_order=act)
    x = synthetic.activations(M, K, seed=77)
    mod = _module_for(layer)
    assert mod.kmap is not None and mod.kinv is not None
    say(f"decode ragged {kernel} K={K} N={N} gs={gs} act={act} M={M}")
    assert_gemm_close(_gemm_raw(mod, x.to(DEV), DOT), _oracle_out(layer, x), f"ragged dot K={K}")


@pytest.mark.parametrize("kernel", ["stream", "tile"])
def test_decode_regime_gathers_through_kmap(kernel, decode_kernel):
    """The decode kernel gathers act-order activations through kmap itself:
    kinv is optional, and with or without it the result is the same."""
    from onecomp_runtime import kernels, synthetic

    decode_kernel(kernel)
    layer = synthetic.gptq_layer(1024, 64, seed=78, act_order=True)
    mod = _module_for(layer)
    x = synthetic.activations(1, 1024, seed=79).to(DEV)
    say(f"decode without kinv ({kernel})")
    out = kernels.int4_gemm(x, mod.tiled(), in_features=1024, kmap=mod.kmap, regime=DOT)
    assert_gemm_close(out, _oracle_out(layer, x.cpu()), "decode without kinv")
    with_kinv = kernels.int4_gemm(x, mod.tiled(), in_features=1024, kmap=mod.kmap, kinv=mod.kinv, regime=DOT)
    assert_gemm_close(with_kinv, _oracle_out(layer, x.cpu()), "decode with kinv")
    auto = kernels.int4_gemm(x, mod.tiled(), in_features=1024, kmap=mod.kmap)
    assert torch.equal(out, auto)


# -- split-item decode kernel (act-order without kinv; K beyond the LDS of the
# whole-tile kernel): K split over workgroups, partials summed in split order by
# the last workgroup of each tile group (device-scope counters that reset). ---
@pytest.fixture
def split_kernel(decode_kernel):
    decode_kernel("split")


def _split_gemv(mod, x, bias=None):
    from onecomp_runtime import kernels

    return kernels.int4_gemm(x, mod.tiled(), in_features=mod.in_features, kmap=mod.kmap, bias=bias, regime=DOT)


@pytest.mark.parametrize("K,N", [(5120, 5120), (17408, 5120), (5120, 1024), (1040, 200), (2048, 17408)])
@pytest.mark.parametrize("M", [1, 2])
def test_split_gemv_matches_oracle(K, N, M, split_kernel):
    from onecomp_runtime import synthetic

    kw = dict(seed=90 + K + M, act_order=True)
    if K == 1040:
        kw = dict(seed=91, groupsize=26)  # padded groups: kmap holds -1 rows
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer)
    x = synthetic.activations(M, K, seed=92)
    say(f"split gemv K={K} N={N} M={M}")
    assert_gemm_close(_split_gemv(mod, x.to(DEV)), _oracle_out(layer, x), f"split gemv K={K} N={N} M={M}")


@pytest.mark.parametrize("M", [1, 2])
def test_split_gemv_one_hot_bit_exact(M, split_kernel):
    from onecomp_runtime import synthetic

    K, N = 4096, 320
    layer = synthetic.gptq_layer(K, N, seed=93, act_order=True)
    mod = _module_for(layer)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    wd = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16", layer.v1)
    rng = np.random.default_rng(2)
    for rep in range(3):
        ks = rng.choice(K, M, replace=False)
        x = torch.zeros((M, K), dtype=torch.bfloat16)
        x[torch.arange(M), torch.from_numpy(ks)] = 1.0
        say(f"split gemv one-hot M={M} rep={rep}")
        assert np.array_equal(bits16(_split_gemv(mod, x.to(DEV))), oracle_bits(wd[:, ks].T, torch.bfloat16))


def test_split_gemv_bias_fp16_deterministic_and_graph(split_kernel):
    from onecomp_runtime import synthetic

    K, N = 8192, 1024
    layer = synthetic.gptq_layer(K, N, seed=94, act_order=True)
    mod16 = _module_for(layer, torch.float16)
    x = synthetic.activations(1, K, seed=95, dtype=torch.float16)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(96)).to(torch.float16)
    say("split gemv fp16 + bias")
    out = _split_gemv(mod16, x.to(DEV), bias.to(DEV))
    assert_gemm_close(out, _oracle_out(layer, x, "f16", bias), "split gemv fp16 bias")
    for rep in range(5):
        assert torch.equal(_split_gemv(mod16, x.to(DEV), bias.to(DEV)), out), f"rep {rep} differs"
    # Graph replays reuse the counters: each replay must match the eager result.
    xd, bd = x.to(DEV), bias.to(DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = _split_gemv(mod16, xd, bd)
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, out), f"graph replay {rep} differs"
        assert torch.equal(_split_gemv(mod16, xd, bd), out)


@pytest.mark.parametrize("M", [1, 2])
def test_decode_beyond_whole_tile_lds(M):
    """K = 65536 fits neither the whole-tile kernel's activation staging nor,
    for M = 2, the stream kernel's: the automatic choice still serves it
    (stream kernel for M = 1, split kernel for M = 2)."""
    from onecomp_runtime import synthetic

    K, N = 65536, 96
    layer = synthetic.gptq_layer(K, N, seed=97)
    mod = _module_for(layer)
    x = synthetic.activations(M, K, seed=98)
    say(f"decode K=65536 M={M}")
    out = mod(x.to(DEV))
    assert_gemm_close(out, _oracle_out(layer, x), f"decode K=65536 M={M}")


# -- stream decode kernel (layers with 256..1536 tiles of 16 columns): each
# workgroup streams an equal range of (tile, 4 K steps) units; a tile cut by a
# range boundary is finished by the second of its two workgroups, which swaps
# in its fp32 partial and gets the first's back (64-bit cells that reset). ---
@pytest.mark.parametrize("K,N,kind", [
    (96, 4096, "plain"),      # 3 K steps (unit = whole tile, lanes past the end): one tile per workgroup
    (160, 4104, "actorder"),  # 5 K steps, 257 tiles with a half tile: cut tiles
    (64, 24576, "plain"),     # 1536 tiles of one unit: 6 tiles per workgroup
    (128, 20000, "kmap"),     # act-order gathered through kmap (no kinv), ragged last tile
    (17408, 5120, "actorder"),
    (5120, 17408, "kmap"),
    (4096, 5120, "plain"),
    (1040, 4104, "gs26"),     # padded groups: zero rows in the staged activations
])
@pytest.mark.parametrize("M", [1, 2])
def test_stream_gemv_range_cuts(K, N, kind, M, decode_kernel):
    from onecomp_runtime import kernels, synthetic

    decode_kernel("stream")
    kw = dict(seed=120 + K % 97 + N % 89)
    if kind in ("actorder", "kmap"):
        kw["act_order"] = True
    if kind == "gs26":
        kw["groupsize"] = 26
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer)
    x = synthetic.activations(M, K, seed=121)
    say(f"stream gemv K={K} N={N} kind={kind} M={M}")
    kinv = None if kind == "kmap" else mod.kinv
    out = kernels.int4_gemm(x.to(DEV), mod.tiled(), in_features=K, kmap=mod.kmap, kinv=kinv, regime=DOT)
    assert_gemm_close(out, _oracle_out(layer, x), f"stream gemv K={K} N={N} {kind} M={M}")


def test_stream_gemv_deterministic_and_graph(decode_kernel):
    """Cut tiles finished through the swap cells: repeated calls and graph
    replays (which reuse the cells) give identical bits."""
    from onecomp_runtime import synthetic

    decode_kernel("stream")
    K, N = 5120, 4104
    layer = synthetic.gptq_layer(K, N, seed=122, act_order=True)
    mod16 = _module_for(layer, torch.float16)
    x = synthetic.activations(2, K, seed=123, dtype=torch.float16)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(124)).to(torch.float16)
    xd, bd = x.to(DEV), bias.to(DEV)
    say("stream gemv fp16 + bias, repeated")
    out = _gemm_bias(mod16, xd, bd)
    assert_gemm_close(out, _oracle_out(layer, x, "f16", bias), "stream gemv fp16 bias")
    for rep in range(5):
        assert torch.equal(_gemm_bias(mod16, xd, bd), out), f"rep {rep} differs"
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = _gemm_bias(mod16, xd, bd)
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, out), f"graph replay {rep} differs"
        assert torch.equal(_gemm_bias(mod16, xd, bd), out)


def _gemm_bias(mod, x, bias):
    from onecomp_runtime import kernels

    return kernels.int4_gemm(x, mod.tiled(), in_features=mod.in_features, kmap=mod.kmap, kinv=mod.kinv, bias=bias,
                             regime=DOT)


@pytest.mark.parametrize("M", [1, 2])
def test_decode_kernels_agree(M, decode_kernel):
    """The three decode kernels compute the same products (fp32 sums in
    different orders): each within the tolerance of the oracle and close to
    one another."""
    from onecomp_runtime import synthetic

    K, N = 5120, 5120
    layer = synthetic.gptq_layer(K, N, seed=125, act_order=True)
    mod = _module_for(layer)
    x = synthetic.activations(M, K, seed=126).to(DEV)
    ref = _oracle_out(layer, x.cpu())
    outs = {}
    for kernel in ("stream", "tile", "split"):
        decode_kernel(kernel)
        say(f"decode kernels agree: {kernel} M={M}")
        outs[kernel] = _gemm_raw(mod, x, DOT)
        assert_gemm_close(outs[kernel], ref, kernel)
    for kernel in ("tile", "split"):
        diff = (outs[kernel].float() - outs["stream"].float()).abs().max().item()
        assert diff <= 2e-2 * outs["stream"].float().abs().max().item(), (kernel, diff)


@pytest.mark.parametrize("regime", [DOT, SPLITK, TILED])
@pytest.mark.parametrize("M", [1, 2])
def test_small_m_bias_all_regimes(regime, M):
    """Bias epilogue and act-order on every regime that takes a decode batch."""
    from onecomp_runtime import synthetic
    from onecomp_runtime.layers import PackedGPTQLinear

    K, N = 2048, 1536
    layer = synthetic.gptq_layer(K, N, seed=74, act_order=True)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    mod = PackedGPTQLinear(K, N, layer.qweight.to(DEV), layer.scales.to(DEV), layer.qzeros.to(DEV),
                           g_idx=layer.g_idx.to(DEV), bias=bias.to(DEV), groupsize=32)
    x = synthetic.activations(M, K, seed=75)
    say(f"small-M bias regime={regime} M={M}")
    assert_gemm_close(_gemm_raw(mod, x.to(DEV), regime), _oracle_out(layer, x, bias=bias.float()),
                      f"regime {regime} M={M}")


# -- stream kernel, MFMA form (3 <= M <= 16 chosen automatically when the
# activation rows fit in LDS): one v_mfma_f32_16x16x32 per K step after a 4 x 4
# transpose of the loaded octets across the wave's 16-lane rows. -------------
def _uses_stream(mod, M):
    """True when the automatic plan takes the stream kernel (its workspace is
    exactly the counter area: no gathered activations, no partials)."""
    from onecomp_runtime import _hip

    w = mod.tiled()
    nbytes = _hip.gemm_workspace_bytes(M, w.N, w.k_phys, w.group_rows, mod.kmap is not None, AUTO)
    return nbytes == 512 * 1024


@pytest.mark.parametrize("M,K,N,kind", [
    (16, 2048, 16400, "plain"),     # 4 tiles per workgroup and a ragged one
    (8, 5120, 5120, "actorder"),    # decode M=8 layers
    (8, 5120, 17408, "actorder"),
    (3, 160, 4104, "actorder"),     # 5 K steps, cut tiles, a ragged tile
    (5, 96, 4112, "plain"),         # 3 K steps: lanes past the tile's end
    (12, 1040, 16392, "gs26"),      # padded groups, a ragged tile
    (4, 4096, 3200, "plain"),       # 200 tiles: one workgroup per tile
    (4, 128, 20000, "kmap"),        # gathered through kmap (no kinv)
    (16, 2048, 8208, "gs128"),
    (9, 64, 24592, "plain"),        # 6 tiles per workgroup
])
def test_stream_mfma_matches_oracle(M, K, N, kind, decode_kernel):
    from onecomp_runtime import kernels, synthetic

    decode_kernel("stream")
    kw = dict(seed=130 + K % 97 + N % 89 + M)
    if kind in ("actorder", "kmap"):
        kw["act_order"] = True
    if kind == "gs26":
        kw["groupsize"] = 26
    if kind == "gs128":
        kw["groupsize"] = 128
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer)
    assert _uses_stream(mod, M)
    x = synthetic.activations(M, K, seed=131)
    say(f"stream mfma K={K} N={N} kind={kind} M={M}")
    kinv = None if kind == "kmap" else mod.kinv
    out = kernels.int4_gemm(x.to(DEV), mod.tiled(), in_features=K, kmap=mod.kmap, kinv=kinv)
    assert_gemm_close(out, _oracle_out(layer, x), f"stream mfma K={K} N={N} {kind} M={M}")


@pytest.mark.parametrize("kind", ["gs32_v1", "v2", "actorder", "gs26", "gs128", "fp16", "bf16_scales"])
@pytest.mark.parametrize("M", [4, 16])
def test_stream_mfma_one_hot_bit_exact(kind, M, decode_kernel):
    """Factored scale and zero on the MFMA form reproduce dequantized rows exactly."""
    from onecomp_runtime import synthetic

    decode_kernel("stream")
    K, N = 1024, 16400
    kw = dict(seed=132)
    dtype = torch.float16 if kind == "fp16" else torch.bfloat16
    if kind == "v2":
        kw["v1"] = False
    if kind == "actorder":
        kw["act_order"] = True
    if kind == "gs26":
        K, kw["groupsize"] = 1040, 26
    if kind == "gs128":
        kw["groupsize"] = 128
    if kind == "bf16_scales":
        kw["scale_dtype"] = torch.bfloat16
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer, dtype)
    assert _uses_stream(mod, M)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    wd = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16" if dtype == torch.bfloat16 else "f16", layer.v1)
    rng = np.random.default_rng(3)
    for rep in range(2):
        ks = rng.choice(K, M, replace=False)
        x = torch.zeros((M, K), dtype=dtype)
        x[torch.arange(M), torch.from_numpy(ks)] = 1.0
        say(f"stream mfma one-hot kind={kind} M={M} rep={rep}")
        out = _gemm_raw(mod, x.to(DEV), AUTO)
        assert np.array_equal(bits16(out), oracle_bits(wd[:, ks].T, dtype))


def test_stream_mfma_deterministic_graph_and_whole_tile_agree(decode_kernel):
    """Repeated calls and graph replays give identical bits; the whole-tile
    MFMA kernel (stream off) computes the same products."""
    from onecomp_runtime import synthetic

    decode_kernel("stream")
    K, N, M = 5120, 4104, 8
    layer = synthetic.gptq_layer(K, N, seed=133, act_order=True)
    mod16 = _module_for(layer, torch.float16)
    assert _uses_stream(mod16, M)
    x = synthetic.activations(M, K, seed=134, dtype=torch.float16)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(135)).to(torch.float16)
    xd, bd = x.to(DEV), bias.to(DEV)
    say("stream mfma fp16 + bias, repeated")
    out = _gemm_bias_auto(mod16, xd, bd)
    assert_gemm_close(out, _oracle_out(layer, x, "f16", bias), "stream mfma fp16 bias")
    for rep in range(3):
        assert torch.equal(_gemm_bias_auto(mod16, xd, bd), out), f"rep {rep} differs"
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = _gemm_bias_auto(mod16, xd, bd)
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, out), f"graph replay {rep} differs"
        assert torch.equal(_gemm_bias_auto(mod16, xd, bd), out)
    decode_kernel("tile")
    assert not _uses_stream(mod16, M)
    say("whole-tile MFMA kernel, same call")
    tile = _gemm_bias_auto(mod16, xd, bd)
    diff = (tile.float() - out.float()).abs().max().item()
    assert diff <= 2e-2 * out.float().abs().max().item(), diff


def _gemm_bias_auto(mod, x, bias):
    from onecomp_runtime import kernels

    return kernels.int4_gemm(x, mod.tiled(), in_features=mod.in_features, kmap=mod.kmap, kinv=mod.kinv, bias=bias)


# -- stream kernel over activation rows in global memory (3 <= M <= 16, rows
# beyond LDS, a tile count that whole tiles would spread unevenly): exact
# dequantization, MFMAs accumulated across K steps, no staging. ---------------
@pytest.mark.parametrize("M,K,N,kind", [
    (4, 17408, 5120, "plain"),
    (8, 17408, 5120, "actorder"),   # decode M=8 layer (rows gathered first)
    (16, 5120, 17408, "actorder"),
    (16, 8224, 4112, "plain"),      # 257 K steps (units past the tile's end), a ragged tile
    (12, 16384, 4112, "gs128"),
    (3, 20000, 5120, "kmap"),       # act-order without kinv
    (8, 5120, 1024, "actorder"),    # 64 tiles: two workgroups per tile (half-tile ranges)
    (5, 4096, 2000, "plain"),       # 125 tiles, a ragged last tile, half-tile ranges
])
def test_stream_global_rows_matches_oracle(M, K, N, kind, decode_kernel):
    from onecomp_runtime import kernels, synthetic

    decode_kernel("global")
    kw = dict(seed=140 + K % 97 + N % 89 + M)
    if kind in ("actorder", "kmap"):
        kw["act_order"] = True
    if kind == "gs128":
        kw["groupsize"] = 128
    layer = synthetic.gptq_layer(K, N, **kw)
    mod = _module_for(layer)
    if mod.kmap is None:
        assert _uses_stream(mod, M)  # the counter area alone: the stream kernel, no gathered rows
    x = synthetic.activations(M, K, seed=141)
    say(f"stream global rows K={K} N={N} kind={kind} M={M}")
    kinv = None if kind == "kmap" else mod.kinv
    out = kernels.int4_gemm(x.to(DEV), mod.tiled(), in_features=K, kmap=mod.kmap, kinv=kinv)
    assert_gemm_close(out, _oracle_out(layer, x), f"stream global K={K} N={N} {kind} M={M}")


@pytest.mark.parametrize("M", [4, 16])
def test_stream_global_rows_one_hot_bit_exact(M, decode_kernel):
    from onecomp_runtime import synthetic

    decode_kernel("global")
    K, N = 4096, 4112
    layer = synthetic.gptq_layer(K, N, seed=142)
    mod = _module_for(layer)
    assert _uses_stream(mod, M)
    qw, sc, qz, g_idx = layer_oracle_inputs(layer)
    wd = O.dequant_gptq(qw, sc, qz, g_idx, K, N, "bf16", layer.v1)
    rng = np.random.default_rng(7)
    for rep in range(2):
        ks = rng.choice(K, M, replace=False)
        x = torch.zeros((M, K), dtype=torch.bfloat16)
        x[torch.arange(M), torch.from_numpy(ks)] = 1.0
        say(f"stream global one-hot M={M} rep={rep}")
        out = _gemm_raw(mod, x.to(DEV), AUTO)
        assert np.array_equal(bits16(out), oracle_bits(wd[:, ks].T, torch.bfloat16))
    # deterministic across calls and equal to the whole-tile kernel within tolerance
    x = synthetic.activations(M, K, seed=143).to(DEV)
    a = _gemm_raw(mod, x, AUTO)
    assert torch.equal(_gemm_raw(mod, x, AUTO), a)
    decode_kernel("tile")
    assert not _uses_stream(mod, M)
    b = _gemm_raw(mod, x, AUTO)
    assert (a.float() - b.float()).abs().max().item() <= 2e-2 * a.float().abs().max().item()
