"""Recomputes the table of the engine's expf (oracle/llmk_oracle.c EXP_TAB,
llm-rs_amd/csrc/llmk_numerics.h kExpTab) from the mathematics.

glibc's expf (sysdeps/ieee754/flt-32/e_expf.c, >= 2.28) scales 2^(k/32) from
a table of 2^(i/32), i = 0..31, each correctly rounded to double and stored
as its bit pattern less (i << 47), so that adding (k << 47) puts k >> 5 into
the exponent field.  This script evaluates 2^(i/32) to 80 decimal digits and
rounds to double; tests/test_oracle_math.py checks that both sources hold
these words.  Run: python oracle/gen_constants.py
"""
import struct
from decimal import Decimal, getcontext


def exp_table():
    getcontext().prec = 80
    ln2 = Decimal(2).ln()
    words = []
    for i in range(32):
        v = (ln2 * i / 32).exp()
        d = float(v)  # Decimal -> float rounds to nearest (ties to even)
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        words.append((bits - (i << 47)) & 0xFFFFFFFFFFFFFFFF)
    return words


if __name__ == "__main__":
    for i, w in enumerate(exp_table()):
        print(f"{i:2d}  0x{w:016x}")
