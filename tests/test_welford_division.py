"""The quotient identity of the tile encoder's Welford step for sealed blocks
(csrc/k4_encode.hip, step_c): for integers 1 <= n <= 256 and finite doubles
delta, RN(delta / n) == fma(delta, y_hi, RN(delta * y_lo)) with
y_hi = RN(1 / n) and y_lo = RN(fma(-y_hi, n, 1) / n).  The torch CPU
var_mean that the encoder restates divides by n once per step
(codec.py:200-210), so the encoder's statistics stay bit-exact only if this
holds for every delta.  Checked here in C (gcc, IEEE doubles, fma from libm)
on random deltas of every exponent range the encoder meets and on deltas
built to put delta / n next to a rounding midpoint."""
import os
import subprocess
import textwrap

import pytest

SRC = textwrap.dedent(r"""
    #include <math.h>
    #include <stdint.h>
    #include <stdio.h>
    #include <string.h>
    static uint64_t s = 0x9e3779b97f4a7c15ull;
    static uint64_t rnd(void) { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; }
    static double from_bits(uint64_t b) { double d; memcpy(&d, &b, 8); return d; }
    int main(void) {
        long bad = 0, checked = 0;
        for (int n = 1; n <= 256; ++n) {
            const double dn = (double)n, yh = 1.0 / dn, yl = fma(-yh, dn, 1.0) / dn;
            for (int i = 0; i < 40000; ++i) {
                double d;
                uint64_t r = rnd();
                if (i % 4 == 0) {
                    /* any sign and mantissa, exponents 2^-300 .. 2^300 */
                    d = ldexp(1.0 + (double)(r >> 12) * 0x1p-52, (int)(rnd() % 601) - 300);
                } else if (i % 4 == 1) {
                    /* a product k * n +- small: delta / n near integers and halves */
                    const double k = (double)(int64_t)(rnd() % 2000001) - 1000000.0;
                    d = (k + 0.5 * (double)(rnd() & 1)) * dn;
                    d = nextafter(d, (r & 1) ? INFINITY : -INFINITY);
                } else if (i % 4 == 2) {
                    /* the midpoint of two doubles times n, then the neighbours of the result */
                    const double q = from_bits((rnd() & 0x000fffffffffffffull) | 0x3ff0000000000000ull);
                    const double m = q + ldexp(1.0, -53);            /* not representable: rounds */
                    d = m * dn;
                    for (int k = (int)(r % 3); k > 0; --k) d = nextafter(d, INFINITY);
                } else {
                    /* bf16-valued inputs minus a running mean of the encoder's range */
                    const double x = (double)from_bits(((rnd() & 0xffffull) << 48) & 0xfff0000000000000ull);
                    d = x - from_bits((r & 0x800fffffffffffffull) | (((rnd() % 64) + 992) << 52));
                }
                if (r & 2) d = -d;
                if (!isfinite(d)) continue;
                const double want = d / dn, got = fma(d, yh, d * yl);
                ++checked;
                if (memcmp(&want, &got, 8) != 0 && !(want == 0.0 && got == 0.0)) {
                    if (bad < 5) printf("mismatch n=%d d=%a want=%a got=%a\n", n, d, want, got);
                    ++bad;
                }
            }
        }
        printf("checked %ld bad %ld\n", checked, bad);
        return bad != 0;
    }
""")


def test_sealed_block_welford_division_is_the_ieee_quotient(tmp_path):
    c = tmp_path / "div.c"
    exe = tmp_path / "div"
    c.write_text(SRC)
    try:
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(c), "-lm"], check=True,
                       capture_output=True, text=True)
    except (OSError, subprocess.CalledProcessError) as e:
        pytest.skip(f"gcc unavailable: {e}")
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bad 0" in r.stdout


# The remainder correction of the general Welford step (k4_encode_kernel for
# rows of any length, k4_encode_tile's table path): y = RN(1 / n),
# q0 = RN(delta y), r = fma(-q0, n, delta) (exact), q = fma(r, y, q0).  Checked
# for every n <= 4096 and random n up to 2^24 (rows of any token count the
# encoders take) with the same delta generators.
SRC_REM = SRC.replace("for (int n = 1; n <= 256; ++n) {", """for (int k = 1; k <= 4096 + 3000; ++k) {
            const int n = k <= 4096 ? k : 4097 + (int)(rnd() % ((1u << 24) - 4097));""").replace(
    "for (int i = 0; i < 40000; ++i) {", "for (int i = 0; i < (k <= 256 ? 4000 : 600); ++i) {").replace(
    "const double want = d / dn, got = fma(d, yh, d * yl);",
    "const double q0 = d * yh, rr = fma(-q0, dn, d), want = d / dn, got = fma(rr, yh, q0); (void)yl;")


# The reciprocal of the general Welford step for rows of up to 2^24 tokens
# (csrc/k4_encode.hip, iq_rcp_small_int): y0 = the float reciprocal of n, then
# twice y = fma(y, fma(-n, y, 1), y).  The hardware float reciprocal is within
# 1 ulp; every start from 4 ulp below to 4 ulp above RN_f32(1 / n) is checked
# against the IEEE double 1.0 / n, for every n from 1 to 2^24.
SRC_RCP = textwrap.dedent(r"""
    #include <math.h>
    #include <stdio.h>
    #include <string.h>
    int main(void) {
        long bad = 0, checked = 0;
        for (unsigned n = 1; n <= (1u << 24); ++n) {
            const double d = (double)n, want = 1.0 / d;
            const float f0 = 1.0f / (float)n;
            float lo = f0;
            for (int k = 0; k < 4; ++k) lo = nextafterf(lo, 0.0f);
            float f = lo;
            for (int p = -4; p <= 4; ++p, f = nextafterf(f, INFINITY)) {
                double y = (double)f;
                y = fma(y, fma(-d, y, 1.0), y);
                y = fma(y, fma(-d, y, 1.0), y);
                ++checked;
                if (memcmp(&y, &want, 8) != 0) {
                    if (bad < 5) printf("mismatch n=%u p=%d got=%a want=%a\n", n, p, y, want);
                    ++bad;
                }
            }
        }
        printf("checked %ld bad %ld\n", checked, bad);
        return bad != 0;
    }
""")


def test_small_integer_reciprocal_is_correctly_rounded(tmp_path):
    c = tmp_path / "rcp.c"
    exe = tmp_path / "rcp"
    c.write_text(SRC_RCP)
    try:
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(c), "-lm"], check=True,
                       capture_output=True, text=True)
    except (OSError, subprocess.CalledProcessError) as e:
        pytest.skip(f"gcc unavailable: {e}")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checked 150994944 bad 0" in r.stdout, r.stdout


def test_remainder_corrected_welford_division_is_the_ieee_quotient(tmp_path):
    assert SRC_REM != SRC and "fma(rr, yh, q0)" in SRC_REM and "4096 + 3000" in SRC_REM
    c = tmp_path / "rem.c"
    exe = tmp_path / "rem"
    c.write_text(SRC_REM)
    try:
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(c), "-lm"], check=True,
                       capture_output=True, text=True)
    except (OSError, subprocess.CalledProcessError) as e:
        pytest.skip(f"gcc unavailable: {e}")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bad 0" in r.stdout
