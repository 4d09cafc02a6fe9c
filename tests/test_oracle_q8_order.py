"""The q8_1 path's Q4_K row dot: per-sub-block fp32 terms and their pairwise sum.

The GPU kernels that form gate/up (whose SiLU-GLU output is quantized to q8_1
again) reproduce this order bit for bit, so a q8_1 value of h can never round
the other way between the device and the oracle. What pins the oracle here:
  - hand-computed known answers whose result depends on the summation tree
    (pairwise 5, sequential 3, exact 6) and on the fused multiply-add in the
    term (16777215 fused, 16777214 with two roundings);
  - a rounding-error bound against the terms' closed form in double on random
    rows at every row width the kernels take.
"""
import numpy as np
import pytest

import kq_synth as S
from kq_synth import Q4_K, Q8_1

F16_ONE = np.array([1.0], np.float16).view(np.uint8)


def _f16(v):
    return np.array([v], np.float16).view(np.uint8)


def _q8_blocks(vals, d8s):
    """q8_1 blocks with given f16 scales and int8 values (s is unused by the dot)."""
    out = np.zeros((len(d8s), 36), np.uint8)
    for k, (d8, v) in enumerate(zip(d8s, vals)):
        out[k, 0:2] = _f16(d8)
        out[k, 4:36] = np.asarray(v, np.int8).view(np.uint8)
    return out.reshape(-1)


def _unit_q4k_block(d=1.0, dmin=0.0):
    """One Q4_K block, every sub-block scale 1 and min 0, nibbles zero."""
    b = np.zeros(144, np.uint8)
    b[0:2] = _f16(d)
    b[2:4] = _f16(dmin)
    b[4:8] = 1        # sc[0..3] = 1
    b[12:16] = 1      # sc[4..7] = 1 (low nibbles), m[4..7] = 0
    return b


def test_pairwise_tree_known_answer(oracle):
    """Terms t = [2^24, 1, 1, 1, -2^24, 1, 1, 1] (sub-block j's term is
    d8_j * isum_j with unit scales and dmin 0). Pairwise:
    (2^24 + 1 -> 2^24 (tie, even)) + 2 = 16777218; (-2^24 + 1) + 2 =
    -16777213; sum 5. A left-to-right fp32 sum gives 3, double gives 6."""
    blk = _unit_q4k_block()
    nib = blk[16:].reshape(4, 32)             # group g: low nibble sub-block 2g, high 2g+1
    nib[0, :] = 0x08                          # sub-block 0: q = 8 everywhere
    nib[0, 0] |= 0x10                         # sub-block 1: q = 1 at value 0
    nib[1, 0] = 0x11                          # sub-blocks 2, 3: q = 1 at value 0
    nib[2, :] = 0x08                          # sub-block 4: q = 8 everywhere
    nib[2, 0] |= 0x10                         # sub-block 5
    nib[3, 0] = 0x11                          # sub-blocks 6, 7
    blk[16:] = nib.reshape(-1)
    one = [1] + [0] * 31
    vals = [[2] * 32, one, one, one, [-2] * 32, one, one, one]
    d8s = [32768.0, 1.0, 1.0, 1.0, 32768.0, 1.0, 1.0, 1.0]
    q8 = _q8_blocks(vals, d8s)
    terms = [oracle.q4K_q8_term(blk, j, q8[36 * j:]) for j in range(8)]
    assert terms == [16777216.0, 1.0, 1.0, 1.0, -16777216.0, 1.0, 1.0, 1.0]
    assert oracle.dot_q4K_q8(blk, q8) == 5.0
    assert oracle.dot_q4K_q8(blk, q8, f64=True) == 6.0


def test_pairwise_split_across_blocks_known_answer(oracle):
    """Two blocks (16 terms): t_0 = 2^24, t_8 = t_15 = 1, the rest 0. The
    halves are summed apart first: 2^24 + (1 + 1) = 16777218, where a
    left-to-right sum loses both ones (16777216)."""
    b0, b1 = _unit_q4k_block(), _unit_q4k_block()
    b0[16:48] = 0x08                          # sub-block 0: q = 8
    b1[16] = 0x01                             # block 1 sub-block 0: q = 1 at value 0
    b1[16 + 96] = 0x10                        # block 1 sub-block 7: q = 1 at value 0
    row = np.concatenate([b0, b1])
    zero, one = [0] * 32, [1] + [0] * 31
    vals = [[2] * 32] + [zero] * 7 + [one] + [zero] * 6 + [one]
    d8s = [32768.0] + [1.0] * 15
    assert oracle.dot_q4K_q8(row, _q8_blocks(vals, d8s)) == 16777218.0


def test_term_is_one_fused_multiply_add(oracle):
    """A = (d*sc)*d8 = (673*1)*257 = 172961, isum = 97: A*isum = 16777217
    (not a float). B = (dmin*m)*d8 = 2^-14*257, xsum = 97: B*xsum =
    24929/16384. fmaf rounds 16777217 - 1.5215... once to 16777215; a
    separate product rounds 16777217 to 16777216 first and ends at 16777214."""
    blk = _unit_q4k_block(d=673.0, dmin=2.0 ** -14)
    blk[4:16] = 0
    blk[4] = 1                                # sc_0 = 1
    blk[8] = 1                                # m_0 = 1
    blk[16] = 0x01                            # sub-block 0: q = 1 at value 0
    q8 = _q8_blocks([[97] + [0] * 31] + [[0] * 32] * 7, [257.0] + [1.0] * 7)
    assert oracle.q4K_q8_term(blk, 0, q8) == 16777215.0
    assert oracle.dot_q4K_q8(blk, q8) == 16777215.0


@pytest.mark.parametrize("cols", [256, 512, 1024, 2048, 4096])
def test_pairwise_dot_error_bound(oracle, cols):
    """|pairwise - closed form| <= (log2(n) + 4) * 2^-24 * sum_j(|A_j isum_j| +
    |B_j xsum_j|), the magnitude bounded element-wise by dequantized weights
    (d*sc*q and dmin*m parts) times |dequantized x|."""
    rng = np.random.default_rng(70 + cols)
    rows = 48
    w = S.matrix(rng, Q4_K, rows, cols)
    q8 = oracle.quantize_q8_1(S.activation(rng, cols))
    xd = np.abs(oracle.dequant(Q8_1, q8, cols).astype(np.float64))
    wb = w.reshape(-1, 144)
    w_scale = wb.copy()
    w_scale[:, 2:4] = 0                        # dmin = 0: d*sc*q
    w_min = wb.copy()
    w_min[:, 0:2] = 0                          # d = 0: -dmin*m
    mag_s = np.abs(oracle.dequant(Q4_K, w_scale.reshape(-1), rows * cols).astype(np.float64)).reshape(rows, cols)
    mag_m = np.abs(oracle.dequant(Q4_K, w_min.reshape(-1), rows * cols).astype(np.float64)).reshape(rows, cols)
    mag = (mag_s + mag_m) @ xd
    n = cols // 32
    rb = cols // 256 * 144
    got = np.array([oracle.dot_q4K_q8(w[r * rb:(r + 1) * rb], q8) for r in range(rows)], np.float64)
    ref = np.array([oracle.dot_q4K_q8(w[r * rb:(r + 1) * rb], q8, f64=True) for r in range(rows)], np.float64)
    bound = (np.log2(n) + 4) * 2.0 ** -24 * mag * 1.01 + np.abs(ref) * 2.0 ** -24
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)
    # the matvec entry point is the same dot row by row
    assert np.array_equal(oracle.matvec_q8(Q4_K, w, rows, cols, q8), got.astype(np.float32))
