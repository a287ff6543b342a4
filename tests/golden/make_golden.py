#!/usr/bin/env python3
"""Generate the golden MXFP4 fixtures in this directory.

The reference ships no tests, fixtures or golden vectors for its kernels, so
these vectors come from a second restatement of the reference rules written
for this purpose: plain Python with exact rational arithmetic (fractions) for
every rounding step and numpy float32 only where the reference computes in
fp32. It shares no code with oracle/mxfp4_oracle.c; tests/test_golden.py
checks that the C oracle and the HIP kernels reproduce every vector.

Rules restated (reference lines):
  * quantize (code/kernel/per_token_quant_mxfp4.cu:151-254): amax = fmaxf over
    |x| seeded with eps (NaN ignored), y_s = 2^ceil(log2(max(fl32(amax/6),
    1e-10f))), byte = log2(y_s) + 127 (inf block -> 126), q = clamp(x / y_s,
    -6, 6) rounded to the nearest E2M1 value, ties to the even code; NaN -> 0xF.
  * dequant (per_token_Mxfp4ToBf16_dequant.cu:22-29, 137-156): bf16(code) *
    bf16(s << 7) in fp32, rounded to bf16 (nearest, ties to even); s = 0 -> 0,
    s = 255 -> inf.
  * rowwise FP8 requant (per_token_Mxfp4ToFp8.cu:162-229): per 128 elements
    g = (uint16)(max of the 4 scale bytes - 6), pattern = bits(code) -
    ((uint16)(g - s_i) << 7) mod 2^16, clamp to +-448, E4M3 nearest-even;
    scale = fp32 bits (uint8)g << 23.

Run: python tests/golden/make_golden.py   (writes the *.json files here)
"""
import json
import math
import os
import struct
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

E2M1 = [Fraction(0), Fraction(1, 2), Fraction(1), Fraction(3, 2), Fraction(2), Fraction(3), Fraction(4), Fraction(6)]


def bf16_value(bits):
    """Exact value of a bf16 pattern: Fraction, or float inf/nan."""
    sign = -1 if bits & 0x8000 else 1
    e, m = (bits >> 7) & 0xFF, bits & 0x7F
    if e == 0xFF:
        return float("nan") if m else sign * float("inf")
    if e == 0:
        return sign * Fraction(m, 1 << 7) * Fraction(1, 1 << 126)
    return sign * (1 + Fraction(m, 128)) * (Fraction(2) ** (e - 127))


def f32(x):
    return np.float32(x)


def f32_exact(v):
    """Exact Fraction of a finite float32 value."""
    return Fraction(float(v))


def e2m1_code(q):
    """Nearest E2M1 code of an exact |q| <= 6, ties to the even code."""
    best = None
    for code, val in enumerate(E2M1):
        d = abs(q - val)
        if best is None or d < best[0] or (d == best[0] and code % 2 == 0):
            best = (d, code)
    return best[1]


def quantize_block(bits, eps=1e-10):
    """32 bf16 patterns -> (scale byte, 16 code bytes)."""
    amax = f32(eps)
    has_inf = False
    for b in bits:
        v = bf16_value(b)
        if isinstance(v, float):
            if math.isnan(v):
                continue  # fmaxf ignores NaN
            has_inf = True
            continue
        amax = max(amax, f32(abs(float(v))))  # |bf16| is exact in float32
    if has_inf:
        scale = 126  # y_s = inf; (int)log2f(inf) saturates, low byte 0x7E
        inv = None
    else:
        z = max(f32(amax) / f32(6.0), f32(1e-10))  # IEEE float32 division
        mant, ex = math.frexp(float(z))  # z = mant * 2^ex, mant in [0.5, 1)
        c = ex - 1 if mant == 0.5 else ex
        scale = (c + 127) & 0xFF
        inv = Fraction(2) ** (-c)
    codes = []
    for b in bits:
        v = bf16_value(b)
        neg = bool(b & 0x8000)
        if isinstance(v, float) or inv is None:
            if isinstance(v, float) and math.isnan(v):
                codes.append(0xF)  # clamp(NaN) = -6
                continue
            if inv is None:
                # x * (1/inf): finite -> +-0, +-inf -> NaN -> -6
                codes.append(0xF if isinstance(v, float) else (0x8 if neg else 0x0))
                continue
        qf = f32(f32(float(v)) * f32(float(inv)))  # fp32 product (exact or underflowing)
        q = f32_exact(qf)
        q = max(Fraction(-6), min(Fraction(6), q))
        code = e2m1_code(abs(q))
        codes.append(code | (8 if (q < 0 or (q == 0 and (neg or math.copysign(1.0, float(qf)) < 0))) else 0))
    out = bytes((codes[2 * j] & 0xF) | ((codes[2 * j + 1] & 0xF) << 4) for j in range(16))
    return scale, out


def bf16_rne(v):
    """Exact value -> bf16 bits, nearest-even (finite or inf)."""
    if v == 0:
        return 0
    sign = 0x8000 if v < 0 else 0
    a = abs(v)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 7)
    n = a / ulp
    fl = math.floor(n)
    r = n - fl
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = fl * ulp
    if val >= Fraction(2) ** 128:
        return sign | 0x7F80
    if val < Fraction(2) ** -126:  # subnormal
        return sign | int(val / Fraction(2) ** -133)
    ee = math.floor(math.log2(val))
    while Fraction(2) ** ee > val:
        ee -= 1
    while Fraction(2) ** (ee + 1) <= val:
        ee += 1
    m = int((val / Fraction(2) ** ee - 1) * 128)
    return sign | ((ee + 127) << 7) | m


def e2m1_bf16_value(nib):
    v = E2M1[nib & 7]
    return -v if nib & 8 else v


def dequant_element(nib, s):
    """bf16 bits of the dequantized element, or None for the unpinned NaN case."""
    if s == 0:
        return 0x8000 if (nib & 8) else 0  # code * 0.0 keeps the sign
    if s == 255:
        if nib & 7 == 0:
            return None  # 0 * inf: NaN payload of the bf16 rounding is unpinned
        return 0xFF80 if nib & 8 else 0x7F80
    if nib & 7 == 0:
        return 0x8000 if nib & 8 else 0  # +-0 times a positive scale keeps its sign
    return bf16_rne(e2m1_bf16_value(nib) * Fraction(2) ** (s - 127))


E4M3 = []  # (value, byte) for the finite non-negative E4M3 values
for e in range(16):
    for m in range(8):
        if e == 15 and m == 7:
            continue
        val = Fraction(m, 8) * Fraction(2) ** -6 if e == 0 else (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7)
        E4M3.append((val, (e << 3) | m))


def e4m3_rne(v):
    """Exact value with |v| <= 448 -> E4M3 byte, nearest-even."""
    a = abs(v)
    best = None
    for val, byte in E4M3:
        d = abs(a - val)
        if best is None or d < best[0] or (d == best[0] and byte % 2 == 0):
            best = (d, byte)
    return best[1] | (0x80 if v < 0 else 0)


def bf16_pattern_value(p):
    """Value of a 16-bit pattern after the reference's float conversion and
    clamp fmaxf(-448, fminf(448, x)) (NaN -> -448)."""
    v = bf16_value(p)
    if isinstance(v, float):
        if math.isnan(v):
            return Fraction(-448)
        return Fraction(448) if v > 0 else Fraction(-448)
    return max(Fraction(-448), min(Fraction(448), v))


def e2m1_bits(nib):
    """bf16 pattern of an E2M1 code (as the reference decodes it)."""
    v = e2m1_bf16_value(nib)
    if v == 0:
        return 0x8000 if nib & 8 else 0
    return bf16_rne(v)


def requant_group(codes64, s4):
    """64 code bytes + 4 scale bytes -> (128 fp8 bytes, fp32 scale bits)."""
    smax = max(s4)
    g16 = (smax - 6) & 0xFFFF
    out = []
    for i in range(128):
        byte = codes64[i // 2]
        nib = (byte >> 4) if i % 2 else (byte & 0xF)
        s_i = s4[i // 32]
        adj = (g16 - s_i) & 0xFFFF
        pat = (e2m1_bits(nib) - ((adj << 7) & 0xFFFF)) & 0xFFFF
        if pat & 0x7FFF == 0:
            out.append(0x80 if pat & 0x8000 else 0x00)  # +-0 passes the clamp with its sign
        else:
            out.append(e4m3_rne(bf16_pattern_value(pat)))
    return bytes(out), (g16 & 0xFF) << 23


def bf16_bits_of(x):
    return int(np.array([x], np.float32).view(np.uint32)[0] >> 16)


def main():
    rng = np.random.default_rng(20261201)
    # ---- quantize blocks
    blocks = []
    for sigma in [1e-30, 1e-12, 1e-3, 0.02, 1.0, 3.0, 100.0, 1e10, 1e30, 3e38]:
        for _ in range(6):
            x = rng.standard_normal(32) * sigma
            x = np.clip(x, -3.3e38, 3.3e38)
            blocks.append([bf16_bits_of(v) for v in x])
    six = 0x40C0
    ties = [0x3E80, 0x3F40, 0x3FA0, 0x3FE0, 0x4020, 0x4060, 0x40A0, 0x40B0]  # 0.25 .. 5.5, the midpoints
    blocks += [
        [0] * 32, [0x8000] * 32, [1, 0x8001, 0x7F, 0x807F] + [0] * 28,
        [0x7FC0] + [0x3F80] * 31, [0x7F80] + [0x3F80, 0xBF80, 0, 0x8000] * 7 + [0x3F80, 0x3F80, 0xFF80],
        [six] + ties * 3 + [0] * 7, [0x40C1] + ties * 3 + [0] * 7, [0x7F7F] + [1] * 31, [0x7F40] + [0x3F80] * 31,
        [0x2F00] * 32, [0x3040] + [0x2FFF] * 31,
    ]
    for e in range(-40, 128, 7):  # anchors 6 * 2^e with a ramp of magnitudes
        anchor = bf16_bits_of(6.0 * 2.0 ** e) if e < 127 else 0x7F7F
        blocks.append([anchor] + [bf16_bits_of((k + 1) * 6.0 * 2.0 ** e / 33.0) ^ (0x8000 if k % 3 == 0 else 0)
                                  for k in range(31)])
    # NaNs after the block maximum, signalling ones included, within one
    # 8-element group: every NaN is ignored by the amax
    blocks += [
        [0x40C8, 0x7F81] + [0x3F80] * 30,
        [0x3F80] * 5 + [0xC0C8, 0xFF81, 0x3F00] + [0x3F80] * 24,
        [0x40C8, 0x7FC0, 0x7F81, 0xFFC0] + [0x3F00] * 28,
        [0x3F00] * 31 + [0x7F81],
    ]
    quant = []
    for b in blocks:
        sc, codes = quantize_block(b)
        quant.append({"x": bytes(struct.pack("<32H", *b)).hex(), "scale": sc, "codes": codes.hex()})
    # ---- dequant: every code under every scale byte
    deq = {}
    for s in range(256):
        deq[str(s)] = [dequant_element(nib, s) for nib in range(16)]
    # ---- rowwise FP8 requant groups
    groups = []
    for k in range(24):
        codes64 = bytes(rng.integers(0, 256, 64, dtype=np.uint8))
        base = int(rng.integers(0, 256))
        spread = [0, 3, 7, 12, 255][k % 5]
        s4 = [max(0, min(255, base - int(rng.integers(0, spread + 1)))) for _ in range(4)]
        if k == 0:
            s4 = [120, 127, 113, 126]  # zero codes with s_i <= max - 7: the -448 wrap
        if k == 1:
            s4 = [3, 0, 5, 1]  # max < 6: g wraps
        if k == 2:
            codes64 = bytes(64)  # all zero codes
        out, sbits = requant_group(codes64, s4)
        groups.append({"codes": codes64.hex(), "scales": s4, "fp8": out.hex(), "scale_bits": sbits})
    with open(os.path.join(HERE, "quant_blocks.json"), "w") as f:
        json.dump({"eps": 1e-10, "blocks": quant}, f, indent=0)
    with open(os.path.join(HERE, "dequant_table.json"), "w") as f:
        json.dump({"note": "bf16 bits of code (0..15) under scale byte; null = unpinned NaN", "table": deq}, f)
    with open(os.path.join(HERE, "fp8_rowwise_groups.json"), "w") as f:
        json.dump({"groups": groups}, f, indent=0)
    print(f"{len(quant)} quantize blocks, 256x16 dequant entries, {len(groups)} FP8 groups")


if __name__ == "__main__":
    main()
