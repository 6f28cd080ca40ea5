"""The byte identities the one-launch kernels pack digits with (common.h pack_digit_bytes),
against the oracle's digit split over every q the digits take. A row whose absmax is 2^F - 1
has exponent F, so sh = 0 and q = trunc(x) = x for integer x: the row of every integer in
(-2^F, 2^F) gives every digit pair the kernels can meet. Balanced digits (F < 15): the high
digit's byte is byte 1 of q + 128, the low digit's byte 0 of q + 128 with its top bit flipped.
Offset digits (F = 15): bytes 1 and 0 of q (the low one flipped), 256 h + l = q - 128, and
q = 128 gives zero digits."""
import numpy as np
import pytest

import oracle


@pytest.mark.parametrize("F", [12, 14, 15])
def test_digit_bytes_match_the_oracle_digits(F):
    q = np.arange(-(1 << F) + 1, 1 << F, dtype=np.int64)
    h, l, cs, sh = oracle.digitize_np(q.astype(np.float32)[None, :], F)
    assert sh[0] == 0
    u = q & 0xFFFFFFFF
    y = u if F == 15 else (u + 128) & 0xFFFFFFFF
    assert np.array_equal(h[0].view(np.uint8), ((y >> 8) & 255).astype(np.uint8))
    assert np.array_equal(l[0].view(np.uint8), ((y & 255) ^ 0x80).astype(np.uint8))
    if F == 15:
        assert int(cs[0]) == int(((q - 128).sum() + (1 << 31)) % (1 << 32) - (1 << 31))
        h0, l0, _, _ = oracle.digitize_np(np.array([[128.0, (1 << 15) - 1]], np.float32), 15)
        assert h0[0, 0] == 0 and l0[0, 0] == 0
