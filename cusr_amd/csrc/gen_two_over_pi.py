"""Prints the bits of 2/pi as 64-bit words for include/cusr_math.h
(cm_two_over_pi): word 0 is zero (bits of weight 2^0 .. 2^-63... none set,
2/pi < 1), word j >= 1 holds the bits of weight 2^-(64(j-1)+1) .. 2^-64j.

pi comes from Machin's formula pi = 16 atan(1/5) - 4 atan(1/239), each atan
summed as an exact integer series at 1,600 fractional bits; 2/pi is then
floor(2^(2P+1) / floor(pi 2^P)). The first word must read 0xA2F9836E4E441529.

    python cusr_amd/csrc/gen_two_over_pi.py
"""
P = 1600
WORDS = 24


def atan_inv(n: int, bits: int) -> int:
    """atan(1/n) * 2^bits, truncated series."""
    one = 1 << (bits + 16)
    term = one // n
    total, k, sign, n2 = term, 1, -1, n * n
    while term:
        term //= n2
        total += sign * (term // (2 * k + 1))
        sign, k = -sign, k + 1
    return total >> 16


def two_over_pi_words() -> list[int]:
    pi = 16 * atan_inv(5, P) - 4 * atan_inv(239, P)
    top = (1 << (2 * P + 1)) // pi            # 2/pi * 2^P
    nbits = 64 * (WORDS - 1)
    stream = top >> (P - nbits)                # bits 1 .. nbits after the point
    return [0] + [(stream >> (nbits - 64 * (j + 1))) & (2 ** 64 - 1) for j in range(WORDS - 1)]


if __name__ == "__main__":
    w = two_over_pi_words()
    assert w[1] == 0xA2F9836E4E441529, hex(w[1])
    for i in range(0, len(w), 3):
        print("    " + ", ".join(f"0x{v:016X}ull" for v in w[i:i + 3]) + ",")
