"""Pins the CPU oracle (oracle/onecomp_oracle.py) before parity tests trust
it as their reference: known answers derived with exact rational arithmetic
(tests/golden/kats.json), torch's own conversions and 16-bit arithmetic (the
reference's arithmetic boundary), format invariants and float64 brute force.
CPU only.
"""
import numpy as np
import pytest
import torch

from oracle import onecomp_oracle as O


def _bits16(vals_f32: np.ndarray, fmt: str) -> np.ndarray:
    if fmt == "bf16":
        return O.f32_to_bf16_bits(vals_f32)
    return np.asarray(vals_f32, dtype=np.float32).astype(np.float16).view(np.uint16)


def _edge_floats() -> np.ndarray:
    rng = np.random.default_rng(1)
    hi = rng.integers(0, 1 << 16, 4000, dtype=np.uint32) << 16
    low = np.concatenate([
        np.full(1000, 0x8000, np.uint32),  # exact ties at bf16
        np.full(1000, 0x7FFF, np.uint32),
        np.full(1000, 0x8001, np.uint32),
        rng.integers(0, 1 << 16, 1000, dtype=np.uint32),
    ])
    bits = hi | low
    specials = np.array([0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000, 0x00000001, 0x807FFFFF,
                         0x00008000, 0x3F808000, 0x3F818000, 0x477FF000, 0x477FEFFF, 0x38800000,
                         0x33800000, 0x33000000, 0x33000001],
                        dtype=np.uint32)
    x = np.concatenate([bits, specials]).view(np.float32)
    return x[~np.isnan(x)]


@pytest.mark.parametrize("fmt,tdtype", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_round_to_matches_torch_conversion(fmt, tdtype):
    x = np.concatenate([_edge_floats(),
                        np.random.default_rng(2).standard_normal(20000).astype(np.float32) * 300])
    mine = O.round_to(x, fmt)
    ref = torch.from_numpy(x).to(tdtype).float().numpy()
    assert np.array_equal(mine.view(np.uint32), ref.view(np.uint32))


def test_round_to_bf16_nan_stays_nan():
    x = np.array([np.nan, -np.nan], dtype=np.float32)
    assert np.isnan(O.round_to(x, "bf16")).all()


def test_unpack_words_known_answers(kats):
    for case in kats["unpack_words"]:
        packed = np.array([[case["word_i32"]]], dtype=np.int32)
        assert O.unpack_rows(packed, 8, 4)[:, 0].tolist() == case["nibbles"]
        assert O.unpack_rows(packed, 4, 8)[:, 0].tolist() == case["bytes"]
        # dropping rows past num_rows (quant_utils.py:28)
        assert O.unpack_rows(packed, 3, 4)[:, 0].tolist() == case["nibbles"][:3]


def test_pack_unpack_round_trip():
    rng = np.random.default_rng(3)
    for K, N in [(8, 8), (37, 16), (1040, 24)]:
        codes = rng.integers(0, 16, (K, N))
        packed = O.pack_rows(codes)
        assert packed.shape == ((K + 7) // 8, N)
        assert np.array_equal(O.unpack_rows(packed, K, 4), codes)
        assert np.array_equal(O.unpack_int_weights(packed, 4, (N, K)), codes.T)
    z = rng.integers(0, 16, (5, 32))
    assert np.array_equal(O.unpack_zeros(O.pack_zeros(z, v1=False), 4, 32), z)
    assert np.array_equal((O.unpack_zeros(O.pack_zeros(z, v1=True), 4, 32) + 1) & 15, z)


def test_v1_zero_known_answers(kats):
    for case in kats["v1_zero"]:
        qz = O.pack_rows(np.array([[case["stored"]] * 8]).T).T  # one word, 8 columns
        qz = np.ascontiguousarray(qz.reshape(1, 1))
        ones = np.ones((1, 8), np.float32)
        w = O.pack_rows(np.zeros((8, 8), np.int64))
        d = O.dequant_gptq(w, ones, qz, np.zeros(8, np.int64), 8, 8, "f32", v1=True)
        assert np.all(d == -case["zero"])


def _one_row_layer(cases):
    """Column n of a K=1 layer holds case n: code w, zero z, scale s."""
    n = len(cases)
    N = (n + 7) // 8 * 8
    codes = np.zeros((1, N), np.int64)
    zeros = np.zeros((1, N), np.int64)
    scales = np.zeros((1, N), np.float32)
    for i, c in enumerate(cases):
        codes[0, i], zeros[0, i] = c["w"], c["z"]
        scales[0, i] = np.array([c["scale_f16_bits"]], np.uint16).view(np.float16)[0]
    return O.pack_rows(codes), scales, O.pack_zeros(zeros, v1=False), N


@pytest.mark.parametrize("fmt", ["bf16", "f16"])
def test_gptq_dequant_known_answers(kats, fmt):
    cases = kats["gptq_dequant"]
    qw, sc, qz, N = _one_row_layer(cases)
    d = O.dequant_gptq(qw, sc, qz, np.zeros(1, np.int64), 1, N, fmt, v1=False)[: len(cases), 0]
    got = _bits16(d, fmt)
    want = np.array([c[f"{fmt}_bits"] for c in cases], np.uint16)
    assert np.array_equal(got, want)


def test_gptq_dequant_special_cases():
    rng = np.random.default_rng(4)
    K, N = 64, 16
    codes = rng.integers(0, 16, (K, N))
    qw = O.pack_rows(codes)
    qz = O.pack_zeros(np.full((2, N), 8), v1=True)
    d = O.dequant_gptq(qw, np.ones((2, N), np.float32), qz, O.default_g_idx(K, 32), K, N, "bf16")
    assert np.array_equal(d, (codes.T - 8).astype(np.float32))
    d0 = O.dequant_gptq(qw, np.zeros((2, N), np.float32), qz, O.default_g_idx(K, 32), K, N, "bf16")
    assert np.all(d0 == 0)


def _rand_layer(rng, K, N, gs, v1=True):
    G = -(-K // gs)
    codes = rng.integers(0, 16, (K, N))
    zeros = rng.integers(0, 16, (G, N))
    scales = (np.abs(rng.standard_normal((G, N))) * 0.01 + 1e-3).astype(np.float16).astype(np.float32)
    return codes, zeros, scales, O.pack_rows(codes), O.pack_zeros(zeros, v1)


def test_act_order_gather_direction():
    """Sorting rows by group turns an act-order layer into a plain one; the
    dequantized columns must follow the sort (catches gathering by the wrong
    index)."""
    rng = np.random.default_rng(5)
    K, N, gs = 96, 16, 32
    codes, zeros, scales, qw, qz = _rand_layer(rng, K, N, gs)
    g_idx = rng.permutation(K) // gs
    perm = np.argsort(g_idx, kind="stable")
    d_act = O.dequant_gptq(qw, scales, qz, g_idx, K, N, "bf16")
    d_sorted = O.dequant_gptq(O.pack_rows(codes[perm]), scales, qz, O.default_g_idx(K, gs), K, N, "bf16")
    assert np.array_equal(d_sorted, d_act[:, perm])
    # and a column of group g uses scales[g]
    k = int(perm[0])
    assert g_idx[k] == 0
    assert np.all(d_act[:, k] == O.round_to(scales[0] * (codes[k] - (zeros[0])).astype(np.float32), "bf16"))


def test_v1_v2_equivalence():
    rng = np.random.default_rng(6)
    K, N = 64, 24
    codes, zeros, scales, qw, qz_v1 = _rand_layer(rng, K, N, 32, v1=True)
    qz_v2 = O.pack_zeros(zeros, v1=False)
    g = O.default_g_idx(K, 32)
    assert np.array_equal(O.dequant_gptq(qw, scales, qz_v1, g, K, N, "bf16", v1=True),
                          O.dequant_gptq(qw, scales, qz_v2, g, K, N, "bf16", v1=False))


def test_linear_matches_float64_bruteforce():
    rng = np.random.default_rng(7)
    M, K, N = 3, 48, 8
    x = O.round_to(rng.standard_normal((M, K)).astype(np.float32), "bf16")
    w = O.round_to(rng.standard_normal((N, K)).astype(np.float32), "bf16")
    b = O.round_to(rng.standard_normal(N).astype(np.float32), "bf16")
    out = O.linear(x, w, b, "bf16")
    for m in range(M):
        for n in range(N):
            exact = sum(float(x[m, k]) * float(w[n, k]) for k in range(K)) + float(b[n])
            ulp = 2.0 ** (np.floor(np.log2(abs(exact))) - 7) if exact else 2.0 ** -133
            assert abs(float(out[m, n]) - exact) <= ulp


def test_gptq_linear_act_order_invariance():
    rng = np.random.default_rng(8)
    M, K, N, gs = 4, 128, 16, 32
    codes, zeros, scales, qw, qz = _rand_layer(rng, K, N, gs)
    g_idx = rng.permutation(K) // gs
    x = O.round_to(rng.standard_normal((M, K)).astype(np.float32), "bf16")
    out = O.gptq_linear(x, qw, scales, qz, g_idx, K, N, "bf16")
    perm = np.argsort(g_idx, kind="stable")
    out_sorted = O.gptq_linear(x[:, perm], O.pack_rows(codes[perm]), scales, qz,
                               O.default_g_idx(K, gs), K, N, "bf16")
    ok, rel, cos = O.gemm_close(out_sorted, out, rel=1e-2)
    assert ok, (rel, cos)


def test_padded_groups_equivalence():
    rng = np.random.default_rng(9)
    M, gs, G, N = 5, 26, 4, 16
    K = gs * G
    codes, zeros, scales, qw, qz = _rand_layer(rng, K, N, gs)
    qw_pad, Kp = O.repack_groups_to_32(qw, K, N, gs)
    assert Kp == 32 * G
    x = O.round_to(rng.standard_normal((M, K)).astype(np.float32), "bf16")
    x_pad = np.zeros((M, Kp), np.float32)
    for g in range(G):
        x_pad[:, 32 * g: 32 * g + gs] = x[:, gs * g: gs * (g + 1)]
    d = O.dequant_gptq(qw, scales, qz, O.default_g_idx(K, gs), K, N, "bf16")
    d_pad = O.dequant_gptq(qw_pad, scales, qz, O.default_g_idx(Kp, 32), Kp, N, "bf16")
    for g in range(G):
        assert np.array_equal(d_pad[:, 32 * g: 32 * g + gs], d[:, gs * g: gs * (g + 1)])
    ok, rel, cos = O.gemm_close(O.linear(x_pad, d_pad), O.linear(x, d), rel=1e-2)
    assert ok, (rel, cos)


def test_rtn_nibble_order(kats):
    for case in kats["rtn_bytes"]:
        assert O.rtn_unpack(np.array([[case["byte"]]], np.uint8), 2)[0].tolist() == case["cols"]
    codes = np.random.default_rng(10).integers(0, 16, (3, 9))
    assert np.array_equal(O.rtn_unpack(O.rtn_pack(codes), 9), codes)


@pytest.mark.parametrize("fmt", ["bf16", "f16"])
def test_rtn_dequant_known_answers(kats, fmt):
    cases = kats["rtn_dequant"]
    n = len(cases)
    q = np.array([[c["w"]] for c in cases], np.uint8)  # col 0 = low nibble
    s = np.array([[c["scale_f16_bits"]] for c in cases], np.uint16).view(np.float16).astype(np.float32)
    z = np.array([[c["zero_f16_bits"]] for c in cases], np.uint16).view(np.float16).astype(np.float32)
    d = O.rtn_dequant(q, s, z, 1, n, fmt)[:, 0]
    assert np.array_equal(_bits16(d, fmt), np.array([c[f"{fmt}_bits"] for c in cases], np.uint16))


@pytest.mark.parametrize("tdtype,fmt", [(torch.bfloat16, "bf16"), (torch.float16, "f16"),
                                         (torch.float32, "f32")])
@pytest.mark.parametrize("G", [1, 4])
def test_rtn_dequant_matches_torch_ops(tdtype, fmt, G):
    """torch's own 16-bit ops in the reference's order (quant_utils.py:91-103)."""
    rng = np.random.default_rng(11)
    rows, K = 64, 32
    q = rng.integers(0, 256, (rows, K // 2)).astype(np.uint8)
    s = torch.from_numpy((np.abs(rng.standard_normal((rows, G))) * 0.05 + 1e-3).astype(np.float16))
    z = torch.from_numpy(rng.uniform(-3, 18, (rows, G)).astype(np.float16))
    w = torch.from_numpy(O.rtn_unpack(q, K)).to(tdtype)
    if G == 1:
        ref = (w - z.to(tdtype)) * s.to(tdtype)
    else:
        ref = ((w.reshape(rows, G, K // G) - z.to(tdtype).unsqueeze(-1))
               * s.to(tdtype).unsqueeze(-1)).reshape(rows, K)
    mine = O.rtn_dequant(q, s.float().numpy(), z.float().numpy(), K, rows, fmt)
    assert np.array_equal(mine, ref.float().numpy())


def test_rtn_dequant_group_mismatch_raises():
    with pytest.raises(RuntimeError):
        O.rtn_dequant(np.zeros((2, 5), np.uint8), np.ones((2, 3), np.float32),
                      np.zeros((2, 3), np.float32), 10, 2, "bf16")


def test_embedding_gather_and_dtype_rule():
    rng = np.random.default_rng(12)
    V, D, G = 50, 32, 2
    q = rng.integers(0, 256, (V, D // 2)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((V, G))) * 0.01 + 1e-3).astype(np.float16).astype(np.float32)
    z = rng.integers(0, 16, (V, G)).astype(np.float32)
    ids = np.array([[3, 0, 49], [-1, 7, 7]])
    out = O.embedding(ids, q, s, z, D, "f16")
    flat = np.array([3, 0, 49, 49, 7, 7])
    assert np.array_equal(out, O.rtn_dequant(q[flat], s[flat], z[flat], D, 6, "f16"))
    assert O.embedding_dtype("bf16") == "bf16" and O.embedding_dtype("i32") == "f16"
    with pytest.raises(IndexError):
        O.embedding(np.array([V]), q, s, z, D, "f16")


def test_moe_matches_per_pair_bruteforce():
    rng = np.random.default_rng(13)
    E, K, N, T, topk = 4, 32, 8, 5, 2
    ws = [O.round_to(rng.standard_normal((N, K)).astype(np.float32), "bf16") for _ in range(E)]
    x = O.round_to(rng.standard_normal((T, K)).astype(np.float32), "bf16")
    ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)])
    y = O.moe(x, ids, ws, "bf16")
    for t in range(T):
        for j in range(topk):
            exact = ws[ids[t, j]].astype(np.float64) @ x[t].astype(np.float64)
            ok, rel, cos = O.gemm_close(y[t * topk + j], exact, rel=1e-2)
            assert ok


def test_gemm_close_rejects_planted_mistakes():
    rng = np.random.default_rng(14)
    ref = rng.standard_normal((16, 32)).astype(np.float32)
    assert O.gemm_close(ref, ref)[0]
    flipped = ref.copy()
    flipped[:, 3] *= -1  # sign error in one column
    assert not O.gemm_close(flipped, ref)[0]
    dropped = ref - ref[:, :1] * 0.05  # a dropped term of a few percent
    assert not O.gemm_close(dropped, ref)[0]
    transposed = ref.T.copy().reshape(ref.shape)  # transposed operand
    assert not O.gemm_close(transposed, ref)[0]


# -- the torch-CPU restatement used for the timed CPU baseline -----------------
@pytest.mark.parametrize("case", ["gs32_v1", "actorder_v1", "gs26_v2", "gs128_8bit"])
def test_cpu_paths_dequant_matches_oracle(case):
    """oracle.cpu_paths dequantizes bit for bit like the numpy oracle."""
    import torch

    from oracle import cpu_paths as C

    rng = np.random.default_rng(hash(case) % 1000)
    K, N, gs, wbits, v1 = 200, 48, 32, 4, True
    if case == "gs26_v2":
        gs, v1 = 26, False
    if case == "gs128_8bit":
        gs, wbits = 128, 8
    G = (K + gs - 1) // gs
    codes = rng.integers(0, 1 << wbits, (K, N))
    zeros = rng.integers(0, 1 << wbits, (G, N))
    scales = (np.abs(rng.standard_normal((G, N))) * 0.01 + 1e-3).astype(np.float16)
    g = rng.permutation(K) // gs if case == "actorder_v1" else O.default_g_idx(K, gs)
    qw, qz = O.pack_rows(codes, wbits), O.pack_zeros(zeros, v1, wbits)
    for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "f16"), (torch.float32, "f32")):
        got = C.dequant_gptq(torch.from_numpy(qw), torch.from_numpy(scales), torch.from_numpy(qz),
                             torch.from_numpy(g), K, N, dt, v1, wbits)
        ref = O.dequant_gptq(qw, scales.astype(np.float32), qz, g, K, N, name, v1, wbits)
        assert np.array_equal(got.float().numpy(), ref), (case, name)


@pytest.mark.parametrize("G", [1, 4])
def test_cpu_paths_rtn_and_gemm_match_oracle(G):
    import torch

    from oracle import cpu_paths as C

    rng = np.random.default_rng(G)
    K, N, M = 128, 40, 9
    q = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    s = (np.abs(rng.standard_normal((N, G))) * 0.05 + 1e-3).astype(np.float16)
    z = rng.uniform(-2, 17, (N, G)).astype(np.float16)
    for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "f16")):
        got = C.rtn_dequant(torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(z), K, dt)
        ref = O.rtn_dequant(q, s.astype(np.float32), z.astype(np.float32), K, N, name)
        assert np.array_equal(got.float().numpy(), ref)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(G)).to(dt)
        lin = C.PackedRTN(torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(z), K, dt)
        ok, rel, cos = O.gemm_close(lin(x).float().numpy(), O.rtn_linear(x.float().numpy(), q, s.astype(np.float32),
                                                                         z.astype(np.float32), K, N, name))
        assert ok and torch.equal(lin.eager()(x), lin(x)), (rel, cos)
    ids = torch.from_numpy(rng.integers(0, N, 17))
    emb = C.embedding(ids, torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(z), K)
    assert emb.dtype == torch.float16
    assert np.array_equal(emb.float().numpy(), O.embedding(ids.numpy(), q, s.astype(np.float32),
                                                           z.astype(np.float32), K, "f16"))


def test_cpu_paths_gptq_linear_matches_oracle():
    import torch

    from oracle import cpu_paths as C

    rng = np.random.default_rng(11)
    K, N, M = 256, 64, 7
    codes, zeros = rng.integers(0, 16, (K, N)), rng.integers(0, 16, (K // 32, N))
    scales = (np.abs(rng.standard_normal((K // 32, N))) * 0.01 + 1e-3).astype(np.float16)
    g = rng.permutation(K) // 32
    qw, qz = O.pack_rows(codes), O.pack_zeros(zeros, True)
    bias = rng.standard_normal(N).astype(np.float32)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    lin = C.PackedGPTQ(torch.from_numpy(qw), torch.from_numpy(scales), torch.from_numpy(qz), torch.from_numpy(g),
                       K, N, torch.bfloat16, True, torch.from_numpy(bias))
    ref = O.gptq_linear(x.float().numpy(), qw, scales.astype(np.float32), qz, g, K, N, "bf16", True, bias=bias)
    ok, rel, cos = O.gemm_close(lin(x).float().numpy(), ref)
    assert ok, (rel, cos)
    assert torch.equal(lin.eager()(x), lin(x))


# -- DSV4 uint8 packing (layers/dsv4_packed_linear.py:22-56) ---------------------
def test_dsv4_byte_order_known_answers(kats):
    for rec in kats["dsv4_bytes"]:
        b = np.array([[rec["byte"]]], np.uint8)
        assert O.dsv4_unpack(b, 2, 4)[0].tolist() == rec["codes2"]
        assert O.dsv4_unpack(b, 4, 2)[0].tolist() == rec["codes4"]


@pytest.mark.parametrize("fmt", ["bf16", "f16"])
def test_dsv4_dequant_known_answers(kats, fmt):
    for rec in kats["dsv4_dequant"]:
        wb = rec["wbits"]
        per = 8 // wb
        codes = np.zeros((1, per), np.int64)
        codes[0, 0] = rec["q"]
        z = np.array([[rec["zero_f16_bits"]]], np.uint16).view(np.float16).astype(np.float32)
        s = np.array([[rec["scale_f16_bits"]]], np.uint16).view(np.float16).astype(np.float32)
        got = O.dequant_dsv4(O.dsv4_pack(codes, wb), s, z, wb, per, per, fmt)[0, 0]
        want = rec[f"{fmt}_bits"]
        assert (int(O.f32_to_bf16_bits(np.float32(got).reshape(1))[0]) if fmt == "bf16" else
                int(np.float32(got).astype(np.float16).view(np.uint16))) == want, rec


@pytest.mark.parametrize("wbits", [2, 4])
def test_dsv4_pack_round_trip_and_orientation(wbits):
    rng = np.random.default_rng(wbits)
    out_f, k, gs = 24, 100, 32
    codes = rng.integers(0, 1 << wbits, (out_f, k))
    packed = O.dsv4_pack(codes, wbits)
    assert packed.shape == (out_f, (k + 8 // wbits - 1) // (8 // wbits))
    assert np.array_equal(O.dsv4_unpack(packed, wbits, k), codes)
    G = (k + gs - 1) // gs
    s = (np.abs(rng.standard_normal((G, out_f))) * 0.02 + 1e-4).astype(np.float16).astype(np.float32)
    z = rng.uniform(0, 1 << wbits, (G, out_f)).astype(np.float16).astype(np.float32)
    a = O.dequant_dsv4(packed, s, z, wbits, gs, k, "bf16")
    b = O.dequant_dsv4(packed, s.T.copy(), z.T.copy(), wbits, gs, k, "bf16")
    assert np.array_equal(a, b)
    # brute force per element
    n, kk = 5, 77
    want = O.round_to(np.float32(np.float32(codes[n, kk] - z[kk // gs, n]) * s[kk // gs, n]), "bf16")
    assert a[n, kk] == want


@pytest.mark.parametrize("stride,dilation,pad", [(1, 1, 0), (2, 1, 3), (3, 2, 4)])
def test_conv_oracles_match_torch_float64(stride, dilation, pad):
    import torch

    rng = np.random.default_rng(stride * 10 + dilation)
    B, C, Co, L, k = 2, 5, 6, 23, 4
    x = rng.standard_normal((B, C, L)).astype(np.float32)
    w = rng.standard_normal((Co, C, k)).astype(np.float32)
    b = rng.standard_normal(Co).astype(np.float32)
    T = (L + 2 * pad - dilation * (k - 1) - 1) // stride + 1
    got = O.conv1d(x, w, b, stride, dilation, pad, T, "f32")
    ref = torch.nn.functional.conv1d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                     torch.from_numpy(b).double(), stride, pad, dilation).numpy()
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)
    wt = rng.standard_normal((C, Co, k)).astype(np.float32)
    for op in (0, stride - 1):
        L_out = (L - 1) * stride - 2 * pad + dilation * (k - 1) + op + 1
        got = O.conv_transpose1d(x, wt, b, stride, dilation, pad, L_out, "f32")
        ref = torch.nn.functional.conv_transpose1d(torch.from_numpy(x).double(), torch.from_numpy(wt).double(),
                                                   torch.from_numpy(b).double(), stride, pad, op, 1,
                                                   dilation).numpy()
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_conv_quantizer_and_nibbles_host():
    """Host helpers of the packed conv layers: nibble order (the RTN order),
    and the RTN conv quantizer reconstructs within half a step."""
    import torch

    from onecomp_runtime.layers import pack_int4_nibbles, quantize_conv_weight, unpack_int4_nibbles

    codes = torch.randint(0, 16, (7, 13), generator=torch.Generator().manual_seed(0))
    packed = pack_int4_nibbles(codes)
    assert np.array_equal(packed.numpy(), O.rtn_pack(codes.numpy()))
    assert torch.equal(unpack_int4_nibbles(packed, 13).long(), codes)
    w = torch.randn(6, 64, generator=torch.Generator().manual_seed(1))
    w[2] = 0.0
    for gs in (32, -1, 48):
        q, s, z, cols = quantize_conv_weight(w, groupsize=gs)
        G = 2 if gs == 32 else 1
        assert cols == 64 and s.shape == (6, G) and s.dtype == torch.float16 and z.dtype == torch.float16
        wd = O.rtn_dequant(q.numpy(), s.float().numpy(), z.float().numpy(), 64, 6, "f32")
        step = np.repeat(s.float().numpy(), 64 // G, axis=1)
        assert (np.abs(wd - w.numpy()) <= 0.5 * step + 2e-3 * np.abs(w.numpy()) + 1e-3).all()
        assert (wd[2] == 0).all()
