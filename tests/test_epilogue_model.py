"""CPU model of the GEMM epilogue's quad-transposed stores (pyasc_amd/csrc/gemm_common.h:
quad_transpose_b16, quad_transpose_b32, store_wave_tile).

The model restates the lane exchanges with the DPP quad permutations and v_perm_b32
byte selection as the device executes them, for all 64 lanes of a wave, and checks
that every element of a wave's 128x128 block is written exactly once, to its own
(row, column), for both the 16-bit and the 32-bit form."""
import numpy as np
import pytest

LANES = np.arange(64)


def dpp_quad(v, pattern):
    """v_mov_b32 with a DPP quad_perm: lane 4q+i reads lane 4q+pattern[i]."""
    src = (LANES & ~3) + np.array(pattern)[LANES & 3]
    return v[src]


def xor1(v):
    return dpp_quad(v, [1, 0, 3, 2])


def xor2(v):
    return dpp_quad(v, [2, 3, 0, 1])


def perm(a, b, sel):
    """v_perm_b32: byte i of the result is byte (sel >> 8i) & 0xff of {a:b} (b in bytes 0-3)."""
    a, b = a.astype(np.uint64), b.astype(np.uint64)
    both = (a << np.uint64(32)) | b
    out = np.zeros_like(a)
    for i in range(4):
        s = np.uint64((sel >> (8 * i)) & 0xFF)
        out |= ((both >> (s * np.uint64(8))) & np.uint64(0xFF)) << np.uint64(8 * i)
    return out.astype(np.uint32)


def quad_transpose_b16(d0, d1):
    t = LANES & 3
    hi2 = (t & 2) != 0
    recv = xor2(np.where(hi2, d0, d1))
    d0 = np.where(hi2, recv, d0)
    d1 = np.where(hi2, d1, recv)
    odd = (t & 1) != 0
    r = xor1(np.where(odd, perm(d1, d0, 0x05040100), perm(d1, d0, 0x07060302)))
    e0, e1 = perm(r, d0, 0x05040100), perm(r, d1, 0x07060100)
    o0, o1 = perm(d0, r, 0x07060100), perm(d1, r, 0x07060302)
    return np.where(odd, o0, e0), np.where(odd, o1, e1)


def quad_transpose_b32(v):
    t = LANES & 3
    hi2 = (t & 2) != 0
    s0 = xor2(np.where(hi2, v[0], v[2]))
    s1 = xor2(np.where(hi2, v[1], v[3]))
    a0, a1 = np.where(hi2, s0, v[0]), np.where(hi2, s1, v[1])
    a2, a3 = np.where(hi2, v[2], s0), np.where(hi2, v[3], s1)
    odd = (t & 1) != 0
    r0 = xor1(np.where(odd, a0, a1))
    r1 = xor1(np.where(odd, a2, a3))
    return [np.where(odd, r0, a0), np.where(odd, a1, r0), np.where(odd, r1, a2), np.where(odd, a3, r1)]


def mfma_block_value(i, j, r, tag_bits):
    """The value lane l holds in register r of block (i, j): a tag of its (row, col) in the
    wave's 128x128 block (column l%32, row 8*(r/4) + 4*(l/32) + r%4)."""
    row = i * 32 + 8 * (r // 4) + 4 * (LANES // 32) + r % 4
    col = j * 32 + (LANES & 31)
    tag = row * 128 + col
    return (tag & ((1 << tag_bits) - 1)).astype(np.uint32), row, col


@pytest.mark.parametrize("out_bytes", [2, 4])
def test_store_wave_tile_writes_every_element_once_in_place(out_bytes):
    written = np.full((128, 128), -1, dtype=np.int64)
    t, q, h = LANES & 3, (LANES & 31) >> 2, LANES >> 5
    for i in range(4):
        for g in range(4):
            row = i * 32 + g * 8 + h * 4 + t
            for j in range(4):
                col0 = j * 32 + 4 * q
                vals = [mfma_block_value(i, j, 4 * g + k, 16 if out_bytes == 2 else 32)[0] for k in range(4)]
                if out_bytes == 2:
                    d0, d1 = quad_transpose_b16(vals[0] | (vals[1] << 16), vals[2] | (vals[3] << 16))
                    out = [d0 & 0xFFFF, d0 >> 16, d1 & 0xFFFF, d1 >> 16]
                else:
                    out = quad_transpose_b32(vals)
                for k in range(4):
                    for lane in range(64):
                        assert written[row[lane], col0[lane] + k] == -1, "element written twice"
                        written[row[lane], col0[lane] + k] = out[k][lane]
    expected = (np.arange(128)[:, None] * 128 + np.arange(128)[None, :])
    if out_bytes == 2:
        expected = expected & 0xFFFF
    np.testing.assert_array_equal(written, expected)


def test_rows_leave_in_consecutive_instructions():
    # for fixed (i, g) the four j-stores of a lane cover 16 consecutive columns in 4-column steps of
    # the same row, so each 128-column row segment leaves in four back-to-back instructions
    q = (LANES & 31) >> 2
    cols = np.stack([j * 32 + 4 * q for j in range(4)])
    assert set(np.unique(cols)) == set(range(0, 128, 4))
