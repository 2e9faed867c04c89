"""The Philox4x32-10 checker against the algorithm's published known-answer vectors (the Random123 distribution's
test vectors for 10 rounds), and the Box-Muller pairs' invariants."""
import math

from philox_ref import normals, philox4x32_10


def test_philox_known_answers():
    assert philox4x32_10((0, 0, 0, 0), (0, 0)) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert philox4x32_10((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0)) == [
        0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]
    # a planted mistake (the two multipliers swapped) fails the first vector
    import philox_ref
    m0, m1 = philox_ref.M0, philox_ref.M1
    try:
        philox_ref.M0, philox_ref.M1 = m1, m0
        assert philox4x32_10((0, 0, 0, 0), (0, 0)) != [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    finally:
        philox_ref.M0, philox_ref.M1 = m0, m1


def test_box_muller_pairs():
    """Each pair (z0, z1) has z0^2 + z1^2 = -2 ln u0 of the block's word, and the first 4000 normals have mean and
    variance within 5 standard errors of 0 and 1."""
    z = normals(4000, seed=12345, stream_id=1)
    w = philox4x32_10((0, 0, 1, 0), (12345, 0))
    assert abs(z[0] ** 2 + z[1] ** 2 + 2 * math.log(((w[0] >> 8) + 0.5) * 2.0 ** -24)) < 1e-9
    n = len(z)
    mean = sum(z) / n
    var = sum((x - mean) ** 2 for x in z) / n
    assert abs(mean) < 5 / math.sqrt(n) and abs(var - 1) < 5 * math.sqrt(2 / n)
