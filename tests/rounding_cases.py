"""Edge cases of the fp32 -> bf16 output rounding, with hand-derived bits.

A bf16 GEMV with K = 8, x = [1, 1, 1, 0.5, 0, ...] and zero bias computes,
for a row [w0, w1, w2, w3, 0, ...], the exact fp32 sum w0 + w1 + w2 + w3 / 2
(every partial sum below is exact in fp32), so the expected output is the
round-to-nearest-even bf16 of that sum, written out here by hand.  The last
row holds a NaN weight and must give NaN.
"""
import numpy as np

SUB = 2.0 ** -133          # smallest bf16 subnormal
MAX = (2 - 2 ** -7) * 2.0 ** 127  # largest finite bf16 (0x7F7F)

ROWS = [  # (w0, w1, w2, w3), expected bf16 bits
    ((1, 2 ** -8, 0, 0), 0x3F80),              # tie; the even neighbour is below
    ((1 + 2 ** -7, 2 ** -8, 0, 0), 0x3F82),    # tie; the even neighbour is above
    ((1, 2 ** -8, 2 ** -16, 0), 0x3F81),       # just above a tie
    ((-1, -(2 ** -8), 0, 0), 0xBF80),          # negative tie
    ((MAX, 2.0 ** 119, 0, 0), 0x7F80),         # tie above the largest finite -> inf
    ((MAX, 2.0 ** 118, 0, 0), 0x7F7F),         # below that tie
    ((0, 0, 0, SUB), 0x0000),                  # 2^-134: tie between 0 and 2^-133
    ((SUB, 0, 0, SUB), 0x0002),                # 1.5 * 2^-133: tie, even above
    ((1, 0, 0, 0), 0x3F80),
]


def gemv_inputs(orc):
    """(W bf16 [N, K], x bf16 [K], bias bf16 [N], expected bits [N-1], N, K)."""
    N, K = len(ROWS) + 1, 8
    W = np.zeros((N, K), np.float32)
    for n, (w, _) in enumerate(ROWS):
        W[n, :4] = w
    W[N - 1, 0] = np.nan
    Wb = orc.f32_to_bf16(W)
    assert np.array_equal(orc.bf16_to_f32(Wb)[: N - 1], W[: N - 1]), "inputs must be bf16-exact"
    x = orc.f32_to_bf16(np.array([1, 1, 1, 0.5, 0, 0, 0, 0], np.float32))
    bias = np.zeros(N, np.uint16)
    want = np.array([e for _, e in ROWS], np.uint16)
    return Wb, x, bias, want, N, K
