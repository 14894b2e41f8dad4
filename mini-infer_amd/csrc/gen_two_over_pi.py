"""Writes the 2/pi table of rope_sincos.h (kTwoOverPiMod4): for e = 1..104,
Y_e = (2^e * 2/pi) mod 4 as three non-overlapping 53-bit chunks
(bits 2^1 .. 2^-51, 2^-52 .. 2^-104, 2^-105 .. 2^-157), each exact in fp64.

pi comes from Machin's formula pi = 16 atan(1/5) - 4 atan(1/239), summed in
integer fixed point with 64 guard bits; the table needs 2/pi to
104 + 2 + 157 = 263 fractional bits.  Usage: python gen_two_over_pi.py
"""

FRAC = 600  # fixed-point fraction bits of the pi computation


def atan_inv(n: int, bits: int) -> int:
    """atan(1/n) * 2^bits, by its alternating series."""
    one = 1 << bits
    total, term, k, sign = 0, one // n, 1, 1
    n2 = n * n
    while term:
        total += sign * (term // k)
        term //= n2
        k += 2
        sign = -sign
    return total


def two_over_pi_fixed(bits: int) -> int:
    g = bits + 64
    pi = 16 * atan_inv(5, g) - 4 * atan_inv(239, g)
    return ((2 << (2 * g)) // pi) >> 64  # 2/pi * 2^bits


def table():
    K = 157  # fraction bits kept per entry
    top = two_over_pi_fixed(FRAC)
    rows = []
    for e in range(1, 105):
        y = ((top << e) >> (FRAC - K)) % (4 << K)  # floor(2^e * 2/pi * 2^K) mod 4 * 2^K
        c0 = y >> (K - 51)                  # 53 bits: 2^1 .. 2^-51
        c1 = (y >> (K - 104)) & ((1 << 53) - 1)
        c2 = y & ((1 << 53) - 1)
        rows.append((c0 * 2.0 ** -51, c1 * 2.0 ** -104, c2 * 2.0 ** -157))
    return rows


if __name__ == "__main__":
    for e, (a, b, c) in enumerate(table(), start=1):
        print(f"    {{{a.hex()}, {b.hex()}, {c.hex()}}},  // e = {e}")
