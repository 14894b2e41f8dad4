// rope_sincos.h -- compact sin/cos of RoPE angles, for host and device.
//
// RoPE angles are float(pos) * inv_freq[i] with inv_freq <= 1, so |a| stays
// far below the range where a general sincosf needs its long (Payne-Hanek)
// argument reduction -- the part that costs a general implementation most of
// its registers.  Both routines here use the published Cody-Waite method
// (W. J. Cody and W. Waite, "Software Manual for the Elementary Functions",
// 1980): k = rint(a * 2/pi), r = a - k*(pi/2) with pi/2 split into three
// constants and one fused multiply-add per constant, then Taylor polynomials
// of sin and cos on |r| <= pi/4 (+ a rounding margin) and the quadrant
// (k mod 4) picks and signs the pair.
//
// fp32 form, valid for |a| <= 2^20 (rope_sincos_f32_ok):
//   P1 = pi/2 rounded to a multiple of 2^-11 and P2 (a multiple of 2^-23) make
//   r1 = a - k*P1 and r2 = r1 - k*P2 exact (|r1| < 4, bits >= 2^-23 for
//   a >= 1; |r2| < 1); only r3 = r2 - k*P3 rounds, so |r - exact| <= ulp(r)/2
//   + |k| * 1.8e-15 (<= 1.2e-9 for |k| <= 2/pi * 2^20).  Taylor truncation:
//   r^11/11! < 2^-29, r^12/12! < 2^-33.  The result is within a few fp32 ulp
//   plus 2^-29.5 absolute of the exact value.
// fp64 form, valid for |a| <= 2^24:
//   Q1 (a multiple of 2^-26) and Q2 (of 2^-52) keep r1, r2 exact; r3 rounds
//   once (2^-54 absolute); Taylor terms through r^17 / r^18 (next term
//   < 2^-63).  The result is within a few fp64 ulp of the exact value.
//
// All arithmetic is written as explicit fmaf/fma or single operations, so a
// host build and a device build round identically whatever their
// floating-point contraction settings.
#pragma once
#include <math.h>

#if defined(__HIPCC__)
#define MI_SINCOS_HD __host__ __device__
#else
#define MI_SINCOS_HD
#endif

namespace mi {

MI_SINCOS_HD inline bool rope_sincos_f32_ok(float a) { return fabsf(a) <= 1048576.0f; }

MI_SINCOS_HD inline void rope_sincos_f32(float a, float* s_out, float* c_out) {
    const float kP1 = 0x1.922p+0f;         // pi/2 to a multiple of 2^-11
    const float kP2 = -0x1.28p-18f;        // next part, a multiple of 2^-23
    const float kP3 = -0x1.777a5cp-25f;    // remainder, rounded to fp32
    const float k = rintf(a * 0x1.45f306p-1f);  // a * 2/pi
    float r = fmaf(-k, kP1, a);
    r = fmaf(-k, kP2, r);
    r = fmaf(-k, kP3, r);
    const float r2 = r * r;
    // sin r = r + r^3 (-1/3! + r^2 (1/5! + r^2 (-1/7! + r^2 / 9!)))
    float ps = fmaf(r2, 2.7557319e-6f, -1.98412698e-4f);
    ps = fmaf(r2, ps, 8.33333333e-3f);
    ps = fmaf(r2, ps, -1.66666667e-1f);
    const float sn = fmaf(r * r2, ps, r);
    // cos r = 1 + r^2 (-1/2! + r^2 (1/4! + r^2 (-1/6! + r^2 (1/8! - r^2/10!))))
    float pc = fmaf(r2, -2.75573192e-7f, 2.48015873e-5f);
    pc = fmaf(r2, pc, -1.38888889e-3f);
    pc = fmaf(r2, pc, 4.16666667e-2f);
    pc = fmaf(r2, pc, -0.5f);
    const float cs = fmaf(r2, pc, 1.0f);
    const int q = static_cast<int>(k) & 3;
    const float s = (q & 1) ? cs : sn;
    const float c = (q & 1) ? sn : cs;
    *s_out = a == 0.0f ? a : ((q & 2) ? -s : s);  // sin(-0) = -0
    *c_out = ((q + 1) & 2) ? -c : c;
}

MI_SINCOS_HD inline void rope_sincos_f64(double a, double* s_out, double* c_out) {
    const double kQ1 = 0x1.921fb54p+0;              // pi/2 to a multiple of 2^-26
    const double kQ2 = 0x1.10b46p-30;               // next part, a multiple of 2^-52
    const double kQ3 = 0x1.1a62633145c07p-54;       // remainder, rounded to fp64
    const double k = rint(a * 0x1.45f306dc9c883p-1);  // a * 2/pi
    double r = fma(-k, kQ1, a);
    r = fma(-k, kQ2, r);
    r = fma(-k, kQ3, r);
    const double r2 = r * r;
    // Taylor coefficients (-1)^n / (2n+1)! and (-1)^n / (2n)!
    double ps = fma(r2, 2.8114572543455206e-15, -7.6471637318198165e-13);
    ps = fma(r2, ps, 1.6059043836821613e-10);
    ps = fma(r2, ps, -2.5052108385441720e-8);
    ps = fma(r2, ps, 2.7557319223985893e-6);
    ps = fma(r2, ps, -1.9841269841269841e-4);
    ps = fma(r2, ps, 8.3333333333333333e-3);
    ps = fma(r2, ps, -1.6666666666666667e-1);
    const double sn = fma(r * r2, ps, r);
    double pc = fma(r2, -1.5619206968586225e-16, 4.7794773323873853e-14);
    pc = fma(r2, pc, -1.1470745597729725e-11);
    pc = fma(r2, pc, 2.0876756987868099e-9);
    pc = fma(r2, pc, -2.7557319223985891e-7);
    pc = fma(r2, pc, 2.4801587301587302e-5);
    pc = fma(r2, pc, -1.3888888888888889e-3);
    pc = fma(r2, pc, 4.1666666666666667e-2);
    pc = fma(r2, pc, -0.5);
    const double cs = fma(r2, pc, 1.0);
    const int q = static_cast<int>(static_cast<long long>(k) & 3);
    const double s = (q & 1) ? cs : sn;
    const double c = (q & 1) ? sn : cs;
    *s_out = a == 0.0 ? a : ((q & 2) ? -s : s);
    *c_out = ((q + 1) & 2) ? -c : c;
}

// Half-width of the interval around an fp32 sin/cos value v from
// rope_sincos_f32 that surely holds RN32(exact): 2^-20 relative (several fp32
// ulp) with a 2^-29 absolute floor for the reduction's absolute error at
// values near zero.  If the interval holds no fp16 rounding boundary, the
// fp16 rounding of v is that of RN32(exact).
MI_SINCOS_HD inline float rope_guard_width(float v) {
    const float d = fabsf(v) * 0x1p-20f;
    return d > 0x1p-29f ? d : 0x1p-29f;
}

}  // namespace mi
