"""Packed int4 Conv1d / ConvTranspose1d (layers/packed_conv.py:123-222) on the
GPU: the GEMM paths (im2col chunks x RTN rows; transposed codes + col2im)
against the oracle's dequant (RTN per-op rounding) and fp32 convolutions.
One-hot inputs make each output a single dequantized weight: bit-exact."""
import numpy as np
import pytest
import torch

from gpu_helpers import assert_gemm_close, bits16, np32, oracle_bits, say
from oracle import onecomp_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _weights(rows, cols, G, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, (rows, cols))
    s = (np.abs(rng.standard_normal((rows, G))) * 0.02 + 1e-3).astype(np.float16)
    z = rng.integers(0, 16, (rows, G)).astype(np.float16)
    return O.rtn_pack(codes), s, z


def _wd(q, s, z, cols, rows, dtype="bf16"):
    return O.rtn_dequant(q, s.astype(np.float32), z.astype(np.float32), cols, rows, dtype)


def _conv(cls, cin, cout, k, G, seed, bias=None, **kw):
    rows = cout if cls.__name__ == "PackedInt4Conv1d" else cin
    cols = (cin if rows == cout else cout) * k
    q, s, z = _weights(rows, cols, G, seed)
    mod = cls(cin, cout, k, qweight=torch.from_numpy(q), scales=torch.from_numpy(s), zeros=torch.from_numpy(z),
              cols=cols, bias=bias, **kw)
    return mod.to(DEV), (q, s, z, rows, cols)


CONV_CASES = [  # cin, cout, k, stride, dilation, padding, pad_mode, causal, G
    (64, 96, 7, 1, 1, 0, "auto", False, 14),
    (32, 48, 4, 2, 1, 0, "auto", True, 1),
    (64, 40, 3, 1, 3, 1, "none", False, 2),
]


@pytest.mark.parametrize("case", range(len(CONV_CASES)))
def test_conv1d_one_hot_bit_exact_and_random(case):
    from onecomp_runtime.layers import PackedInt4Conv1d
    from onecomp_runtime.layers.packed_conv import conv1d_pads

    cin, cout, k, st, dil, pad, mode, causal, G = CONV_CASES[case]
    bias = torch.randn(cout, generator=torch.Generator().manual_seed(case))
    mod, (q, s, z, rows, cols) = _conv(PackedInt4Conv1d, cin, cout, k, G, 20500 + case, stride=st, dilation=dil,
                                       padding=pad, pad_mode=mode, causal=causal)
    B, L = 2, 57
    x = torch.zeros(B, cin, L, dtype=torch.bfloat16)
    x[0, 5, 20] = 1.0
    x[1, cin - 1, 3] = 1.0
    assert mod._fused_ok(x.to(DEV))
    say(f"conv1d one-hot case {case}")
    y = mod(x.to(DEV))
    left, right = conv1d_pads(L, k, st, dil, mode, causal)
    T = (L + left + right + 2 * pad - dil * (k - 1) - 1) // st + 1
    assert y.shape == (B, cout, T)
    w = _wd(q, s, z, cols, rows).reshape(cout, cin, k)
    ref = O.conv1d(np32(x), w, None, st, dil, left + pad, T, "bf16")
    assert np.array_equal(bits16(y), oracle_bits(ref, torch.bfloat16))
    mod_b = PackedInt4Conv1d(cin, cout, k, st, pad, dil, qweight=torch.from_numpy(q), scales=torch.from_numpy(s),
                             zeros=torch.from_numpy(z), cols=cols, bias=bias, pad_mode=mode, causal=causal).to(DEV)
    xr = torch.randn(B, cin, L, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    say(f"conv1d random case {case}")
    ref = O.conv1d(np32(xr), w, O.round_to(bias.numpy(), "bf16"), st, dil, left + pad, T, "bf16")
    assert_gemm_close(mod_b(xr.to(DEV)), ref, f"conv1d case {case}")


WIDE_CASES = [  # cin, cout, k, G, scale dtype: chunks of >= 1024 rows on the large-M kernel (K slices: 1, 2, 3;
    (64, 200, 5, 5, np.float16),  # the last case takes 128-column blocks in 4 slices)
    (256, 200, 4, 8, np.float16),
    (320, 96, 5, 25, "bf16"),
    (512, 256, 4, 16, np.float16),
]


@pytest.mark.parametrize("case", range(len(WIDE_CASES)))
def test_conv1d_large_m_kernel(case, monkeypatch):
    """Conv1d chunks of 1024 or more rows on the tile layout (oc_rtn_tile_prepare
    + the large-M kernel, K slices into fp32 partials): one-hot bit-exact,
    random inputs at GEMM tolerance against the oracle and the tiled kernel;
    non-integral zeros clear the fast flags and keep the tiled kernel."""
    from onecomp_runtime.layers import PackedInt4Conv1d

    cin, cout, k, G, sdt = WIDE_CASES[case]
    cols = cin * k
    q, s, z = _weights(cout, cols, G, 20900 + case)
    if sdt == "bf16":
        s_t = torch.from_numpy(s.astype(np.float32)).to(torch.bfloat16)
        z_t = torch.from_numpy(z.astype(np.float32)).to(torch.bfloat16)
        s32, z32 = s_t.float().numpy(), z_t.float().numpy()
    else:
        s_t, z_t = torch.from_numpy(s), torch.from_numpy(z)
        s32, z32 = s.astype(np.float32), z.astype(np.float32)
    bias = torch.randn(cout, generator=torch.Generator().manual_seed(case))
    mod = PackedInt4Conv1d(cin, cout, k, qweight=torch.from_numpy(q), scales=s_t, zeros=z_t, cols=cols, bias=bias,
                           pad_mode="none").to(DEV)
    w = O.rtn_dequant(q, s32, z32, cols, cout, "bf16").reshape(cout, cin, k)
    B, L = 2, 700
    T = L - k + 1
    x = torch.zeros(B, cin, L, dtype=torch.bfloat16)
    x[0, 3, 17] = 1.0
    x[1, cin - 1, L - 1] = 1.0
    x[1, cin // 2, 400] = 1.0
    xr = torch.randn(B, cin, L, generator=torch.Generator().manual_seed(30 + case)).to(torch.bfloat16)
    ref = O.conv1d(np32(xr), w, O.round_to(bias.numpy(), "bf16"), 1, 1, 0, T, "bf16")
    say(f"conv1d large-M kernel case {case}")
    mod0 = PackedInt4Conv1d(cin, cout, k, qweight=torch.from_numpy(q), scales=s_t, zeros=z_t, cols=cols,
                            pad_mode="none").to(DEV)
    for tdt, odt in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
        y1 = mod0(x.to(tdt).to(DEV))
        assert mod0._tile_cache is not None and mod0._tile_cache[3] == (1, 1)
        wo = O.rtn_dequant(q, s32, z32, cols, cout, odt).reshape(cout, cin, k)
        ref1 = O.conv1d(np32(x), wo, None, 1, 1, 0, T, odt)
        assert np.array_equal(bits16(y1), oracle_bits(ref1, tdt)), odt
    yr = mod(xr.to(DEV))
    assert_gemm_close(yr, ref, f"conv1d large-M case {case}")
    monkeypatch.setenv("ONECOMP_HIP_CONV_WIDE", "0")
    yt = mod(xr.to(DEV))
    monkeypatch.delenv("ONECOMP_HIP_CONV_WIDE")
    assert_gemm_close(yr, yt.float().cpu().numpy(), f"conv1d large-M vs tiled case {case}")
    if case == 0:
        zh = (z.astype(np.float32) + 0.5).astype(np.float16)
        modh = PackedInt4Conv1d(cin, cout, k, qweight=torch.from_numpy(q), scales=s_t, zeros=torch.from_numpy(zh),
                                cols=cols, bias=bias, pad_mode="none").to(DEV)
        say("conv1d large-M kernel, half-integral zeros (tiled kernel)")
        yh = modh(xr.to(DEV))
        assert modh._tile_cache[3] == (0, 0)
        wh = O.rtn_dequant(q, s32, zh.astype(np.float32), cols, cout, "bf16").reshape(cout, cin, k)
        assert_gemm_close(yh, O.conv1d(np32(xr), wh, O.round_to(bias.numpy(), "bf16"), 1, 1, 0, T, "bf16"),
                          "conv1d half-integral zeros")


TCONV_CASES = [  # cin, cout, k, stride, dilation, padding, output_padding, pad_mode, causal, G
    (64, 48, 4, 2, 1, 0, 0, "auto", False, 6),
    (32, 40, 16, 8, 1, 0, 0, "auto", True, 1),
    (64, 24, 3, 1, 2, 1, 0, "none", False, 3),
    (32, 32, 5, 3, 1, 2, 2, "none", False, 4),
]


@pytest.mark.parametrize("case", range(len(TCONV_CASES)))
def test_conv_transpose1d_one_hot_bit_exact_and_random(case):
    from onecomp_runtime.layers import PackedInt4ConvTranspose1d
    from onecomp_runtime.layers.packed_conv import _convtranspose1d_unpad

    cin, cout, k, st, dil, pad, opad, mode, causal, G = TCONV_CASES[case]
    bias = torch.randn(cout, generator=torch.Generator().manual_seed(case))
    kw = dict(stride=st, dilation=dil, padding=pad, output_padding=opad, pad_mode=mode, causal=causal)
    mod, (q, s, z, rows, cols) = _conv(PackedInt4ConvTranspose1d, cin, cout, k, G, 20600 + case, **kw)
    B, L = 2, 31
    x = torch.zeros(B, cin, L, dtype=torch.bfloat16)
    x[0, 3, 10] = 1.0
    x[1, cin - 1, L - 1] = 1.0
    assert mod._fused_ok(x.to(DEV))
    say(f"conv-transpose one-hot case {case}")
    y = mod(x.to(DEV))
    L_out = (L - 1) * st - 2 * pad + dil * (k - 1) + opad + 1
    w = _wd(q, s, z, cols, rows).reshape(cin, cout, k)
    ref = _convtranspose1d_unpad(torch.from_numpy(O.conv_transpose1d(np32(x), w, None, st, dil, pad, L_out, "bf16")),
                                 k, st, mode, causal).numpy()
    assert y.shape == ref.shape
    assert np.array_equal(bits16(y), oracle_bits(ref, torch.bfloat16))
    mod_b = PackedInt4ConvTranspose1d(cin, cout, k, qweight=torch.from_numpy(q), scales=torch.from_numpy(s),
                                      zeros=torch.from_numpy(z), cols=cols, bias=bias, **kw).to(DEV)
    xr = torch.randn(B, cin, L, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    say(f"conv-transpose random case {case}")
    ref = O.conv_transpose1d(np32(xr), w, O.round_to(bias.numpy(), "bf16"), st, dil, pad, L_out, "bf16")
    ref = _convtranspose1d_unpad(torch.from_numpy(ref), k, st, mode, causal).numpy()
    assert_gemm_close(mod_b(xr.to(DEV)), ref, f"conv-transpose case {case}")


TWIDE_CASES = [  # cin, cout, k, stride, G: 1024+ input positions on the large-M kernel (K slices: 1, 1, 2)
    (64, 48, 4, 2, 6),
    (128, 40, 16, 8, 20),
    (512, 24, 8, 4, 6),
]


@pytest.mark.parametrize("case", range(len(TWIDE_CASES)))
def test_conv_transpose1d_large_m_kernel(case, monkeypatch):
    """ConvTranspose1d GEMMs over 1024 or more input positions on the
    transposed tile layout (oc_rtn_tile_prepare_t: per-K-row parameters
    rounded to the activation dtype, one layout per dtype): one-hot
    bit-exact in bf16 and fp16, random inputs at GEMM tolerance against the
    oracle and the tiled kernel; non-integral zeros keep the tiled kernel."""
    from onecomp_runtime.layers import PackedInt4ConvTranspose1d

    cin, cout, k, st, G = TWIDE_CASES[case]
    cols = cout * k
    q, s, z = _weights(cin, cols, G, 21000 + case)
    bias = torch.randn(cout, generator=torch.Generator().manual_seed(case))
    kw = dict(stride=st, pad_mode="none")
    mod0 = PackedInt4ConvTranspose1d(cin, cout, k, qweight=torch.from_numpy(q), scales=torch.from_numpy(s),
                                     zeros=torch.from_numpy(z), cols=cols, **kw).to(DEV)
    mod = PackedInt4ConvTranspose1d(cin, cout, k, qweight=torch.from_numpy(q), scales=torch.from_numpy(s),
                                    zeros=torch.from_numpy(z), cols=cols, bias=bias, **kw).to(DEV)
    B, L = 1, 1100
    L_out = (L - 1) * st + k
    for tdt, odt in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
        w = _wd(q, s, z, cols, cin, odt).reshape(cin, cout, k)
        x = torch.zeros(B, cin, L, dtype=tdt)
        x[0, 3, 10] = 1.0
        x[0, cin - 1, L - 1] = 1.0
        x[0, cin // 2, 700] = 1.0
        say(f"conv-transpose large-M kernel case {case} {odt}")
        y1 = mod0(x.to(DEV))
        assert mod0._tile_cache[tdt][3] == 1
        ref1 = O.conv_transpose1d(np32(x), w, None, st, 1, 0, L_out, odt)
        assert np.array_equal(bits16(y1), oracle_bits(ref1, tdt))
    w = _wd(q, s, z, cols, cin).reshape(cin, cout, k)
    xr = torch.randn(B, cin, L, generator=torch.Generator().manual_seed(40 + case)).to(torch.bfloat16)
    ref = O.conv_transpose1d(np32(xr), w, O.round_to(bias.numpy(), "bf16"), st, 1, 0, L_out, "bf16")
    yr = mod(xr.to(DEV))
    assert_gemm_close(yr, ref, f"conv-transpose large-M case {case}")
    monkeypatch.setenv("ONECOMP_HIP_CONV_WIDE", "0")
    yt = mod(xr.to(DEV))
    monkeypatch.delenv("ONECOMP_HIP_CONV_WIDE")
    assert_gemm_close(yr, yt.float().cpu().numpy(), f"conv-transpose large-M vs tiled case {case}")
    if case == 0:
        zh = (z.astype(np.float32) + 0.5).astype(np.float16)
        modh = PackedInt4ConvTranspose1d(cin, cout, k, qweight=torch.from_numpy(q), scales=torch.from_numpy(s),
                                         zeros=torch.from_numpy(zh), cols=cols, bias=bias, **kw).to(DEV)
        say("conv-transpose large-M kernel, half-integral zeros (tiled kernel)")
        yh = modh(xr.to(DEV))
        assert modh._tile_cache[torch.bfloat16][3] == 0
        wh = _wd(q, s, zh, cols, cin).reshape(cin, cout, k)
        assert_gemm_close(yh, O.conv_transpose1d(np32(xr), wh, O.round_to(bias.numpy(), "bf16"), st, 1, 0, L_out,
                                                 "bf16"), "conv-transpose half-integral zeros")


def test_long_sequences_take_several_chunks():
    """More positions than one workspace chunk holds: chunked im2col rows for
    Conv1d, chunked input positions (accumulated in order) for the transpose."""
    from onecomp_runtime.layers import PackedInt4Conv1d, PackedInt4ConvTranspose1d
    from onecomp_runtime.layers.packed_conv import conv1d_pads

    mod, (q, s, z, rows, cols) = _conv(PackedInt4Conv1d, 64, 96, 7, 14, 20700, pad_mode="auto")
    B, L = 2, 60000  # 120000 output rows; a chunk holds 128 MB / (2 * 448 + 4 * 96) B = 104704 rows
    x = torch.randn(B, 64, L, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    say("conv1d long sequence")
    y = mod(x.to(DEV))
    w = _wd(q, s, z, cols, rows).reshape(96, 64, 7)
    left, right = conv1d_pads(L, 7, 1, 1, "auto", False)
    assert y.shape == (B, 96, L + left + right - 6)
    assert_gemm_close(y, O.conv1d(np32(x), w, None, 1, 1, left, y.shape[-1], "bf16"), "conv1d long")
    tmod, (q, s, z, rows, cols) = _conv(PackedInt4ConvTranspose1d, 64, 96, 4, 8, 20701, stride=2, pad_mode="none")
    Lt = 100000  # a chunk holds 128 MB / (2 * 64 + 4 * 384) B = 80640 positions
    xt = torch.randn(1, 64, Lt, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    say("conv-transpose long sequence")
    yt = tmod(xt.to(DEV))
    wt = _wd(q, s, z, cols, rows).reshape(64, 96, 4)
    L_out = (Lt - 1) * 2 + 4
    assert_gemm_close(yt, O.conv_transpose1d(np32(xt), wt, None, 2, 1, 0, L_out, "bf16"), "conv-transpose long")


def test_grouped_conv_takes_the_dequant_path():
    from onecomp_runtime.layers import PackedInt4Conv1d

    rows, cols = 32, (32 // 4) * 3
    q, s, z = _weights(rows, cols, 1, 20800)
    mod = PackedInt4Conv1d(32, 32, 3, groups=4, qweight=torch.from_numpy(q), scales=torch.from_numpy(s),
                           zeros=torch.from_numpy(z), cols=cols, pad_mode="none").to(DEV)
    x = torch.randn(2, 32, 40, generator=torch.Generator().manual_seed(11)).to(torch.bfloat16)
    assert not mod._fused_ok(x.to(DEV))
    say("grouped conv (dequant path)")
    w = torch.from_numpy(_wd(q, s, z, cols, rows).reshape(32, 8, 3))
    ref = torch.nn.functional.conv1d(x.float(), w, None, 1, 0, 1, 4).to(torch.bfloat16)
    assert_gemm_close(mod(x.to(DEV)), np32(ref), "grouped conv")
    assert np.array_equal(bits16(mod._materialize(torch.bfloat16).reshape(32, -1)),
                          oracle_bits(_wd(q, s, z, cols, rows), torch.bfloat16))


def test_replace_conv_with_packed_model():
    from onecomp_runtime.layers import PackedInt4Conv1d, PackedInt4ConvTranspose1d, replace_conv_with_packed

    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Conv1d(64, 128, 7, padding=3), torch.nn.ELU(),
                                torch.nn.ConvTranspose1d(128, 64, 4, stride=2, padding=1),
                                torch.nn.Conv1d(64, 32, 3, padding=1))
    stats = replace_conv_with_packed(model, groupsize=32, cast_remaining_to=None)
    assert stats["replaced"] == 3 and 0 < stats["ratio"] < 0.2
    assert isinstance(model[0], PackedInt4Conv1d) and isinstance(model[2], PackedInt4ConvTranspose1d)
    x = torch.randn(2, 64, 50, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    ref = x.float()
    for m in model:  # the same layers evaluated from dequantized weights, fp32 on the host
        if isinstance(m, PackedInt4Conv1d):
            w = torch.from_numpy(_wd(m.qweight.numpy(), m.scales.numpy(), m.zeros.numpy(), m.cols,
                                     m.out_channels)).reshape(m.out_channels, m.in_channels, m.kernel_size)
            ref = torch.nn.functional.conv1d(ref, w, m.bias.to(torch.bfloat16).float(), m.stride, m.padding)
        elif isinstance(m, PackedInt4ConvTranspose1d):
            w = torch.from_numpy(_wd(m.qweight.numpy(), m.scales.numpy(), m.zeros.numpy(), m.cols,
                                     m.in_channels)).reshape(m.in_channels, m.out_channels, m.kernel_size)
            ref = torch.nn.functional.conv_transpose1d(ref, w, m.bias.to(torch.bfloat16).float(), m.stride,
                                                       m.padding)
        else:
            ref = m(ref)
        ref = ref.to(torch.bfloat16).float()
    model = model.to(DEV)
    say("replace_conv_with_packed model")
    with torch.no_grad():
        out = model(x.to(DEV))
    assert_gemm_close(out, ref.numpy(), "packed conv model")
