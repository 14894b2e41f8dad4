// CPU check of mini-infer_amd/csrc/rope_sincos.h, the sin/cos the RoPE
// kernels use to build cos/sin tables from positions.  The header is plain
// C++ on the host and is compiled here with -ffp-contract=off; every
// operation in it is an explicit fmaf/fma or a single rounding, so the host
// and device builds produce the same bits.
//
// Claims checked, over a strided sweep of every fp32 angle in [0, 2^20]
// (and negatives), plus every RoPE angle float(p) * inv_freq[i] for
// head_dim 128, theta 1e4 and 1e6, p < 65536:
//   1. the guard interval [v - d, v + d], d = rope_guard_width(v), around the
//      fp32 value v holds RN32(exact) -- exact from libm's double sin/cos;
//   2. the table value the kernels produce (fp32 form, fp64 re-evaluation
//      near an fp16 rounding boundary, fp64 form above 2^20) equals
//      half(RN32(exact)), the oracle's rule, bit for bit -- also at and just
//      beyond 2^24, where the fp64 form changes from Cody-Waite to the
//      Payne-Hanek reduction, and for fp32 angles up to 2^63 (every int64
//      position) and the largest finite fp32;
//   3. the fp64 form stays within 2^-50 relative of long-double sin/cos, on
//      both sides of 2^24 and up to 2^127.
// Exit status 0 and "ALL OK" when every claim holds.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <initializer_list>

#include "mi_oracle.h"
#include "rope_sincos.h"

static float bits_to_float(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static float f16_value(float v) { return mio_f16_to_f32(mio_f32_to_f16(v)); }

static long g_checked = 0, g_guard_fail = 0, g_table_fail = 0, g_fallback = 0;

static void check_angle(float a) {
    double es = sin((double)a), ec = cos((double)a);
    float rs = (float)es, rc = (float)ec;
    float s, c;
    mi::rope_sincos_f32(a, &s, &c);
    bool fast_ok = mi::rope_sincos_f32_ok(a);
    if (fast_ok) {
        for (int t = 0; t < 2; ++t) {
            const float v = t ? c : s, r = t ? rc : rs;
            const float d = mi::rope_guard_width(v);
            if (!(r >= v - d && r <= v + d)) {
                if (g_guard_fail < 5) printf("guard: a=%a v=%a RN32(exact)=%a d=%a\n", a, v, r, d);
                ++g_guard_fail;
            }
        }
    }
    // the kernels' composition (rope.hip, cos_sin_half)
    auto near = [](float v) {
        const float d = mi::rope_guard_width(v);
        return f16_value(v - d) != f16_value(v + d);
    };
    if (!fast_ok || near(c) || near(s)) {
        double sd, cd;
        mi::rope_sincos_any(a, &sd, &cd);
        c = (float)cd;
        s = (float)sd;
        ++g_fallback;
    }
    if (mio_f32_to_f16(c) != mio_f32_to_f16(rc) || mio_f32_to_f16(s) != mio_f32_to_f16(rs)) {
        if (g_table_fail < 5) printf("table: a=%a\n", a);
        ++g_table_fail;
    }
    ++g_checked;
}

int main() {
    for (uint32_t b = 0; b <= 0x49800000u; b += 61) check_angle(bits_to_float(b));
    for (uint32_t b = 0x80000000u; b <= 0xC9800000u; b += 4999) check_angle(bits_to_float(b));
    // above 2^20: the fp64 form alone (positions up to 2^24)
    for (uint32_t b = 0x49800001u; b <= 0x4B800000u; b += 997) check_angle(bits_to_float(b));
    // at and just beyond 2^24 (the Cody-Waite / Payne-Hanek boundary), both signs
    for (uint32_t b = 0x4B7FF000u; b <= 0x4B801000u; ++b) {
        check_angle(bits_to_float(b));
        check_angle(-bits_to_float(b));
    }
    // beyond 2^24: int64 positions (to 2^63) and the rest of the fp32 range
    for (uint32_t b = 0x4B800001u; b <= 0x5F000000u; b += 1009) check_angle(bits_to_float(b));
    for (uint32_t b = 0x5F000001u; b <= 0x7F7FFFFFu; b += 100003) check_angle(bits_to_float(b));
    for (int64_t p : {int64_t{16777216}, int64_t{16777217}, int64_t{16777218}, int64_t{1} << 31,
                      (int64_t{1} << 40) + 12345, int64_t{9223372036854775807}})
        check_angle((float)p);
    for (double theta : {1.0e4, 1.0e6}) {
        for (int i = 0; i < 64; ++i) {
            const float inv = powf((float)theta, -(float)(2 * i) / 128.0f);
            for (int p = 0; p < 65536; ++p) check_angle((float)p * inv);
        }
    }
    double worst64 = 0.0;
    long fp64_checked = 0;
    for (uint32_t b = 0x3f800000u; b <= 0x7F7FFFFFu; b += 40961) {
        const float a = bits_to_float(b);
        double s, c;
        mi::rope_sincos_any(a, &s, &c);
        const long double es = sinl((long double)a), ec = cosl((long double)a);
        // relative error, away from the zeros (where it measures the absolute
        // error of the reduction, 2^-60 or better, not the value)
        if (fabsl(es) > 0x1p-8L) {
            const double rs = (double)(fabsl((long double)s - es) / fabsl(es));
            if (rs > worst64) worst64 = rs;
        }
        if (fabsl(ec) > 0x1p-8L) {
            const double rc = (double)(fabsl((long double)c - ec) / fabsl(ec));
            if (rc > worst64) worst64 = rc;
        }
        ++fp64_checked;
    }
    printf("angles %ld, fp64 re-evaluations %ld (%.3f%%), guard failures %ld, table mismatches %ld, "
           "fp64 worst relative error 2^%.1f over %ld angles to 2^128\n",
           g_checked, g_fallback, 100.0 * g_fallback / g_checked, g_guard_fail, g_table_fail,
           log2(worst64), fp64_checked);
    const bool ok = g_guard_fail == 0 && g_table_fail == 0 && worst64 < 0x1p-50;
    if (ok) printf("ALL OK\n");
    return ok ? 0 : 1;
}
