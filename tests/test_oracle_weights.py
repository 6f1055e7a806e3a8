"""The oracle's GGUF weight dequantizers (or_dequant, src/core/dequant/) pinned on the
reference's own tests (q8_0.rs:121-132, q4_k.rs:155-188, q5_k.rs:231-248, q6_k.rs:208-235),
on scale/min values worked out by hand from q4_k.rs's literal scale bytes, and on closed
forms of each format (element order, offsets, ranges)."""
import numpy as np
import pytest

from oracle import oracle

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 8, 12, 13, 14
ONE, HALF = (0x00, 0x3C), (0x00, 0x38)  # f16 1.0 and 0.5, little endian


def test_q8_0_known_values():
    """q8_0.rs:121-132: scale 1, qs[0] = 10, qs[1] = -5."""
    b = np.zeros(34, np.uint8)
    b[0:2] = ONE
    b[2] = 10
    b[3] = np.uint8(-5 & 0xFF)
    out = oracle.dequant(Q8_0, b, 32)
    assert out[0] == 10.0 and out[1] == -5.0 and (out[2:] == 0).all()
    b[0:2] = HALF
    b[2:] = np.arange(32, dtype=np.int8).view(np.uint8) - 16
    assert np.array_equal(oracle.dequant(Q8_0, b, 32), (np.arange(32) - 16) * 0.5)


def test_q4_0_order_offsets_and_scale():
    """Low nibbles of bytes 0..15 are elements 0..15, high nibbles 16..31, minus 8."""
    b = np.zeros(18, np.uint8)
    b[0:2] = HALF
    b[2:] = (np.arange(16) | ((15 - np.arange(16)) << 4)).astype(np.uint8)
    out = oracle.dequant(Q4_0, b, 32)
    assert np.array_equal(out[:16], (np.arange(16) - 8) * 0.5)
    assert np.array_equal(out[16:], (15 - np.arange(16) - 8) * 0.5)
    assert out.max() == 3.5 and out.min() == -4.0  # 7 * d and -8 * d


def test_q5_0_fifth_bit():
    """q5_0.rs:104-134: 5-bit values 0..31 minus 16; the fifth bit of element e is qh bit e."""
    b = np.zeros(22, np.uint8)
    b[0:2] = ONE
    b[2:6] = np.frombuffer(np.uint32(0x80000001).tobytes(), np.uint8)  # elements 0 and 31
    b[6:] = 0xF0  # low nibbles 0, high nibbles 15
    out = oracle.dequant(Q5_0, b, 32)
    exp = np.array([0 - 16] * 16 + [15 - 16] * 16, np.float32)
    exp[0] += 16
    exp[31] += 16
    assert np.array_equal(out, exp)
    assert out.max() == 15.0 and out.min() == -16.0


SCALES = np.array([0b11000011, 0b01000010, 0b10000001, 0b00000000, 0b00111111, 0b00001111,
                   0b11110000, 0b10101010, 0b01010101, 0b10011001, 0b11111111, 0b00000001], np.uint8)
# worked out by hand from the packing (6-bit scales and mins; j >= 4 take their top bits from
# the top bits of bytes j - 4 and j)
SC = [3, 2, 1, 0, 53, 25, 47, 1]
MN = [63, 15, 48, 42, 5, 9, 63, 32]


@pytest.mark.parametrize("fmt", [Q4_K, Q5_K])
def test_k_scale_min_packing(fmt):
    """q4_k.rs:155-188's scale bytes: with d = 1, dmin = 0 and every quant 1, sub-block j is
    sc_j; with d = 0, dmin = 1 it is -m_j."""
    n = 144 if fmt == Q4_K else 176
    qoff = 16 if fmt == Q4_K else 48
    b = np.zeros(n, np.uint8)
    b[4:16] = SCALES
    b[qoff:] = 0x11
    b[0:2] = ONE
    out = oracle.dequant(fmt, b, 256).reshape(8, 32)
    assert np.array_equal(out, np.repeat(np.array(SC, np.float32)[:, None], 32, 1))
    b[0:4] = (0, 0) + ONE
    out = oracle.dequant(fmt, b, 256).reshape(8, 32)
    assert np.array_equal(out, -np.repeat(np.array(MN, np.float32)[:, None], 32, 1))


def test_q4_k_nibble_layout():
    """Chunk c of 64: its 32 bytes' low nibbles are elements 64c..64c+31, high nibbles the next 32."""
    b = np.zeros(144, np.uint8)
    b[0:2] = ONE
    b[4:8] = 1  # sc = 1 for sub-blocks 0..3, mins 0
    b[8:12] = 0
    b[12:16] = 0x01  # sub-blocks 4..7: sc 1, m 0
    q = (np.arange(128) % 16) | ((15 - np.arange(128) % 16) << 4)
    b[16:] = q.astype(np.uint8)
    out = oracle.dequant(Q4_K, b, 256).reshape(4, 2, 32)
    lo = (np.arange(128) % 16).reshape(4, 32)
    assert np.array_equal(out[:, 0], lo) and np.array_equal(out[:, 1], 15 - lo)


def test_q5_k_high_bit():
    """q5_k.rs:231-248: element i takes bit i // 32 of qh[i % 32] as its fifth bit."""
    b = np.zeros(176, np.uint8)
    b[0:2] = ONE
    b[4:8] = 1
    b[12:16] = 0x01
    b[16] = 0b10101010
    b[16 + 31] = 0b00000001
    out = oracle.dequant(Q5_K, b, 256)
    hot = {31, 32, 96, 160, 224}
    assert all(out[i] == (16.0 if i in hot else 0.0) for i in range(256))


def test_q6_k_structure():
    """q6_k.rs:208-235: d = 1, scales 1, a 6-bit value of 32 is 0; all-zero quants are -32;
    element order: part p of each 128-half takes low (p even) or high nibbles of ql[l] (p < 2)
    or ql[l + 32] and bits 2p of qh."""
    b = np.zeros(210, np.uint8)
    b[208:210] = ONE
    b[192:208] = 1
    b[128] = 0x02
    out = oracle.dequant(Q6_K, b, 256)
    assert out[0] == 0.0 and (out[1:] == -32.0).all()
    b[128] = 0
    b[0] = 0x5A       # ql[0]: element 0 low nibble 10, element 64 high nibble 5
    b[32] = 0x3C      # ql[32]: element 32 low 12, element 96 high 3
    b[128] = 0b11100100  # qh[0]: element 0 bits 0, element 32 bits 1, element 64 bits 2, element 96 bits 3
    b[192 + 2] = 3    # scale of elements 32..47 (part 1, first 16)
    out = oracle.dequant(Q6_K, b, 256)
    assert out[0] == 10 - 32 and out[32] == 3 * (12 + 16 - 32)
    assert out[64] == 5 + 32 - 32 and out[96] == 3 + 48 - 32


def test_f32_f16_and_bad_input():
    w = np.array([1.5, -2.25, 3e-3, 65504.0, -0.0, 7.0, 1e-8, 2.0], np.float32)
    assert np.array_equal(oracle.dequant(F32, w.view(np.uint8), 8), w)
    h = w.astype(np.float16)
    assert np.array_equal(oracle.dequant(F16, h.view(np.uint8), 8), h.astype(np.float32))
    with pytest.raises(ValueError):
        oracle.dequant(Q4_0, np.zeros(18, np.uint8), 16)  # partial block
    with pytest.raises(ValueError):
        oracle.dequant(3, np.zeros(20, np.uint8), 32)  # Q4_1: not a format of the path
