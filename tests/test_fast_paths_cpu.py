"""CPU checks of the closed forms the GPU fast paths rest on, against the
oracle (the reference rule restated operation by operation).

* The quantize's block scale: for a block whose max |x| is the bf16 pattern
  a < 0x7F80, the kernels compute the E8M0 byte as
  max((a - 193) >> 7, c_eps + 127) (arithmetic shift), c_eps being the host's
  exponent of max(eps / 6, 1e-10). The reference computes the scale of
  fmaxf(eps, amax) (code/kernel/per_token_quant_mxfp4.cu:151,185-192).
* The rowwise FP8 requant's byte table: for x = max(s) - s_i <= 11 the
  kernel looks each magnitude up in bytes base - 8 (x - 6) (zero code 0, or
  0xFE when x >= 7) and moves the code's sign to bit 7
  (code/kernel/per_token_Mxfp4ToFp8.cu:162-229 for the rule).

Both are exhaustive over their inputs; a wrong constant, shift or sign
fails them.
"""
import numpy as np
import pytest

EPS_VALUES = [1e-10, 0.0, -1.0, 1e-3, 0.5, 3.0, 1e30]


def host_c_eps(eps, fp4_max=6.0):
    y = np.float32(np.float32(eps) / np.float32(fp4_max))
    z = max(y, np.float32(1e-10))
    b = int(np.array(z, np.float32).view(np.uint32))
    return ((b >> 23) & 0xFF) - 127 + (1 if (b & 0x7FFFFF) else 0)


def kernel_scale_byte(a, c_eps):
    """The kernels' closed form, vectorised over bf16 patterns a."""
    a = a.astype(np.int64)
    return np.maximum((a - 193) >> 7, c_eps + 127)


@pytest.mark.parametrize("eps", EPS_VALUES)
def test_block_scale_closed_form(oracle, eps):
    a = np.arange(0, 0x7F80, dtype=np.uint16)  # every finite non-negative bf16 pattern
    blocks = np.zeros((a.size, 32), np.uint16)
    blocks[:, 5] = a
    blocks[1::2, 17] = a[1::2] | 0x8000  # the same magnitude negative, in half the blocks
    _, scales = oracle.quant_mxfp4(blocks.reshape(-1), eps=eps)
    want = scales.astype(np.int64)
    got = kernel_scale_byte(a, host_c_eps(eps))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"eps={eps}: first mismatch at amax 0x{int(a[bad[0]]):04x}: {got[bad[0]]} vs {want[bad[0]]}"


def kernel_fp8_bytes(code_byte, x):
    """The rowwise requant's fast path for one code byte (two elements) under
    gap x = max(s) - s_i in [0, 11]: the two E4M3 bytes (element 2j, 2j+1)."""
    rep = (8 * x) * 0x01010101
    t_hi = (0x7C787470 - rep) & 0xFFFFFFFF
    lo = (0x6C686058 - rep) & 0xFFFFFFFF
    t_lo = (lo & 0xFFFFFF00) | (0xFE if x >= 7 else 0)
    table = [(t_lo >> (8 * k)) & 0xFF for k in range(4)] + [(t_hi >> (8 * k)) & 0xFF for k in range(4)]
    out = []
    for nib in (code_byte & 0xF, code_byte >> 4):
        out.append(table[nib & 7] ^ (0x80 if nib & 8 else 0))
    return out


def test_requant_fast_table(oracle):
    """Every gap x in 0..11 under every code byte, group maximum 200 (and 3,
    where g = max - 6 wraps below zero)."""
    rows = []
    for smax in (200, 3):
        for x in range(12):
            if x > smax:
                continue
            # one 128-element group: block 0 holds the maximum, blocks 1..3 scale smax - x;
            # 64 code bytes: block 0 zeros, blocks 1..3 all 256 byte values over 5 rows
            for part in range(6):
                q = np.zeros(64, np.uint8)
                vals = (np.arange(48) + 48 * part) % 256
                q[16:64] = vals
                s = np.array([smax, smax - x, smax - x, smax - x], np.uint8)
                rows.append((q, s, x, vals))
    q = np.stack([r[0] for r in rows])
    s = np.stack([r[1] for r in rows])
    out, _ = oracle.mxfp4_to_fp8(q, s)
    for i, (_, _, x, vals) in enumerate(rows):
        got = [b for v in vals for b in kernel_fp8_bytes(int(v), x)]
        want = out[i, 32:128].tolist()
        assert got == want, f"row {i} gap {x}: {got[:8]} vs {want[:8]}"
