"""Derives the 32-entry table of the glibc expf restatement (oracle/sa_oracle.c
sao_expf_glibc, solidattention-repro_amd/csrc/represent.hip expf_glibc):

    tab[i] = bits(2^(i/32) correctly rounded to double) - (i << 47)

(glibc 2.35 sysdeps/ieee754/flt-32/e_exp2f_data.c stores the table this way,
so that adding k << 47 to tab[k % 32] scales 2^((k % 32)/32) by 2^(k div 32)
through the exponent field).  2^(i/32) is evaluated with 80-digit decimal
arithmetic and rounded to the nearest double through an exact fraction.
Test infrastructure: the C and HIP sources hold the table; tests compare them
against this derivation."""
from __future__ import annotations

import struct
from decimal import Decimal, getcontext
from fractions import Fraction


def expf_table() -> list[int]:
    getcontext().prec = 80
    ln2 = Decimal(2).ln()
    out = []
    for i in range(32):
        d = float(Fraction((ln2 * i / 32).exp()))  # float(Fraction) rounds to nearest
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        out.append((bits - (i << 47)) & 0xFFFFFFFFFFFFFFFF)
    return out


if __name__ == "__main__":
    for i in range(0, 32, 4):
        print("    " + ", ".join(f"0x{t:016x}ull" for t in expf_table()[i:i + 4]) + ",")
