"""Writes kats.json: known answers for the packed formats and the dequant
rounding, derived with exact rational arithmetic (fractions.Fraction) and a
round-to-nearest-even written from its definition. Nothing here uses numpy,
torch or the oracle, so the answers pin the oracle independently.

    python tests/golden/make_kats.py    # rewrites tests/golden/kats.json
"""
from __future__ import annotations

import json
import random
import struct
from fractions import Fraction
from pathlib import Path

FORMATS = {"bf16": (8, -126, 127), "f16": (11, -14, 15), "f32": (24, -126, 127)}  # precision p, emin, emax


def rne(v: Fraction, fmt: str) -> Fraction:
    """Nearest value of the binary format (ties to even); overflow -> inf."""
    p, emin, emax = FORMATS[fmt]
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)  # subnormals share the quantum of emin
    quantum = Fraction(2) ** (e - (p - 1))
    q = a / quantum
    lo = q.numerator // q.denominator
    rem = q - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1):
        lo += 1
    r = lo * quantum
    if r >= Fraction(2) ** (emax + 1):
        return sign * Fraction(2) ** (emax + 1)  # stands for +-inf
    return sign * r


def f16_exact(x: float) -> Fraction:
    """Exact value of the fp16 nearest to x (via the struct 'e' codec)."""
    return Fraction(struct.unpack("<e", struct.pack("<e", x))[0])


def f16_bits(v: Fraction) -> int:
    return struct.unpack("<H", struct.pack("<e", float(v)))[0]


def bf16_bits(v: Fraction) -> int:
    return struct.unpack("<I", struct.pack("<f", float(v)))[0] >> 16


def out_bits(v: Fraction, fmt: str) -> int:
    _, _, emax = FORMATS[fmt]
    if abs(v) >= Fraction(2) ** (emax + 1):  # overflowed: +-inf
        inf = 0x7F80 if fmt == "bf16" else 0x7C00
        return inf | (0x8000 if v < 0 else 0)
    return bf16_bits(v) if fmt == "bf16" else f16_bits(v)


def main() -> None:
    rnd = random.Random(20260)
    kats: dict = {}

    # 1. int32 words -> 8 nibbles, value i at bits 4i (unsigned view of the word)
    words = [0x76543210, 0xFEDCBA98, 0x80000000, 0xFFFFFFFF, 0x00000000, 0x0000000F, 0xF0000000,
             0x12345678]
    kats["unpack_words"] = [
        {"word_u32": w, "word_i32": w - (1 << 32) if w >= 1 << 31 else w,
         "nibbles": [(w >> (4 * i)) & 0xF for i in range(8)],
         "bytes": [(w >> (8 * i)) & 0xFF for i in range(4)]}
        for w in words
    ]

    # 2. v1 zero restore: stored -> (stored + 1) mod 16
    kats["v1_zero"] = [{"stored": s, "zero": (s + 1) % 16} for s in range(16)]

    # 3. GPTQ dequant: RNE_out(s * (w - z)), s an fp16 value, exact product
    cases = []
    specials = [(1.0, 15, 8), (1.0, 0, 8), (1.0 + 2 ** -8, 9, 8), (1.0 + 2 ** -8, 11, 8),
                (1.0 + 3 * 2 ** -9, 13, 0), (0.0, 7, 3), (2 ** -20, 15, 0), (65504.0, 15, 0)]
    for s, w, z in specials:
        cases.append((f16_exact(s), w, z))
    for _ in range(200):
        s = f16_exact(abs(rnd.gauss(0, 1)) * 0.01 + 1e-3)
        cases.append((s, rnd.randrange(16), rnd.randrange(16)))
    kats["gptq_dequant"] = [
        {"scale_f16_bits": f16_bits(s), "w": w, "z": z,
         "bf16_bits": out_bits(rne(s * (w - z), "bf16"), "bf16"),
         "f16_bits": out_bits(rne(s * (w - z), "f16"), "f16")}
        for s, w, z in cases
    ]

    # 4. RTN per-op rounding: RNE(RNE(w - RNE(z)) * RNE(s)) in the out dtype,
    #    with non-integer zeros so the intermediate roundings matter.
    rtn = []
    for _ in range(300):
        s = f16_exact(abs(rnd.gauss(0, 1)) * 0.05 + 1e-3)
        z = f16_exact(rnd.uniform(-3, 18))
        w = rnd.randrange(16)
        rec = {"scale_f16_bits": f16_bits(s), "zero_f16_bits": f16_bits(z), "w": w}
        for fmt in ("bf16", "f16"):
            d = rne(w - rne(z, fmt), fmt)
            rec[f"{fmt}_bits"] = out_bits(rne(d * rne(s, fmt), fmt), fmt)
        rtn.append(rec)
    kats["rtn_dequant"] = rtn

    # 5. RTN nibble order: byte j -> (col 2j = low nibble, col 2j+1 = high nibble)
    kats["rtn_bytes"] = [{"byte": b, "cols": [b & 0xF, b >> 4]} for b in (0x00, 0x21, 0xF0, 0x0F, 0xA5, 0xFF)]

    # 6. DSV4 uint8 packing along the in-dim: byte -> 8 // wbits codes, low bits first
    kats["dsv4_bytes"] = [{"byte": b, "codes2": [(b >> (2 * i)) & 3 for i in range(4)],
                           "codes4": [b & 0xF, b >> 4]} for b in (0x00, 0x1B, 0xE4, 0xFF, 0x80, 0x36)]

    # 7. DSV4 dequant (layers/dsv4_packed_linear.py:22-56): in fp32,
    #    d = RNE_f32(q - z), v = RNE_f32(d * s), then RNE to the output type;
    #    z and s fp16 values (z not necessarily an integer; tiny ones make the
    #    fp32 subtraction round).
    dsv4 = []
    special = [(2, 3, 2 ** -14 * (1 + 2 ** -10), 1.0), (4, 15, 2 ** -14 * (1 + 2 ** -10), 3.0 + 2 ** -9),
               (4, 0, 0.5, 1.0), (2, 1, 1.5, 2 ** -24), (4, 7, 7.0, 65504.0)]
    for wb, q, z, s_ in special:
        dsv4.append((wb, q, f16_exact(z), f16_exact(s_)))
    for _ in range(240):
        wb = rnd.choice((2, 4))
        q = rnd.randrange(1 << wb)
        z = f16_exact(rnd.uniform(-1.0, (1 << wb) + 1.0)) if rnd.random() < 0.8 else f16_exact(
            rnd.choice((1, -1)) * 2.0 ** rnd.randrange(-24, -10) * rnd.uniform(1, 2))
        s_ = f16_exact(abs(rnd.gauss(0, 1)) * 0.02 + 1e-4)
        dsv4.append((wb, q, z, s_))
    recs = []
    for wb, q, z, s_ in dsv4:
        v = rne(rne(q - z, "f32") * s_, "f32")
        def signed_bits(fmt):  # a negative value that rounds to zero is -0
            r = out_bits(rne(v, fmt), fmt)
            return r | 0x8000 if v < 0 else r

        recs.append({"wbits": wb, "q": q, "zero_f16_bits": f16_bits(z), "scale_f16_bits": f16_bits(s_),
                     "bf16_bits": signed_bits("bf16"), "f16_bits": signed_bits("f16")})
    kats["dsv4_dequant"] = recs

    out = Path(__file__).with_name("kats.json")
    out.write_text(json.dumps(kats, indent=1))
    print(f"wrote {out} ({sum(len(v) for v in kats.values())} cases)")


if __name__ == "__main__":
    main()
