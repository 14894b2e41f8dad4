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
// fp64 Cody-Waite form (in rope_sincos_any), valid for |a| <= 2^24 (proved below; the
//   proof holds to 2^26, the stated bound keeps a margin):
//   Q1 (a multiple of 2^-26, 27 significant bits) and Q2 (a multiple of
//   2^-52, 20 significant bits) make k*Q1 and k*Q2 exact for |k| < 2^26
//   (at most 26 + 27 bits), and |k| <= 2/pi * 2^24 < 2^24; r1 = a - k*Q1,
//   r2 = r1 - k*Q2 exact (results below 2 on the multiples' grids); r3
//   rounds once (2^-54 absolute); Taylor terms through r^17 / r^18 (next
//   term < 2^-63).  The result is within a few fp64 ulp of the exact value.
// Any fp32 angle (rope_sincos_any): above 2^24 an fp32 a is m * 2^e with an
//   integer m < 2^24 and 1 <= e <= 104, and a * 2/pi mod 4 = m * Y_e mod 4
//   with Y_e = 2^e * 2/pi mod 4 from a table of three 53-bit chunks
//   (gen_two_over_pi.py; 157 fraction bits).  m * chunk0 is split exactly
//   with an fma (77 bits: rounded product + exact error), reduced mod 4
//   exactly, and the rest is summed in fp64 (absolute error < 2^-78);
//   k = rint(t), f = t - k, r = f * pi/2 with pi/2 as two doubles.  This is
//   the published Payne-Hanek reduction (M. Payne and R. Hanek, "Radian
//   reduction for trigonometric functions", SIGNUM Newsletter 18(1), 1983),
//   followed by the fp64 polynomials above.
//
// All arithmetic is written as explicit fmaf/fma or single operations, so a
// host build and a device build round identically whatever their
// floating-point contraction settings.
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

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

// sin and cos of a reduced fp64 argument r (|r| <= pi/4 plus a rounding
// margin) in quadrant q (k mod 4), as (s, c) of the original angle.
MI_SINCOS_HD inline void rope_sincos_quadrant(double r, int q, double* s_out, double* c_out) {
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
    const double s = (q & 1) ? cs : sn;
    const double c = (q & 1) ? sn : cs;
    *s_out = (q & 2) ? -s : s;
    *c_out = ((q + 1) & 2) ? -c : c;
}

// Y_e = 2^e * 2/pi mod 4 for e = 1 .. 104, three 53-bit chunks each
// (gen_two_over_pi.py writes this table).
constexpr double kTwoOverPiMod4[104][3] = {
    {0x1.45f306dc9c882p+0, 0x1.4a7f09d5f47d4p-53, 0x1.a6ee06db14accp-106},  // e = 1
    {0x1.45f306dc9c882p+1, 0x1.4a7f09d5f47d4p-52, 0x1.a6ee06db14accp-105},  // e = 2
    {0x1.17cc1b727220ap+0, 0x1.29fc2757d1f52p-53, 0x1.4ddc0db629599p-105},  // e = 3
    {0x1.17cc1b727220ap+1, 0x1.29fc2757d1f53p-52, 0x1.377036d8a5664p-106},  // e = 4
    {0x1.7cc1b727220a8p-2, 0x1.4fe13abe8fa98p-54, 0x1.377036d8a5664p-105},  // e = 5
    {0x1.7cc1b727220a8p-1, 0x1.4fe13abe8fa9ap-53, 0x1.bb81b6c52b324p-107},  // e = 6
    {0x1.7cc1b727220a8p+0, 0x1.4fe13abe8fa9ap-52, 0x1.bb81b6c52b326p-106},  // e = 7
    {0x1.7cc1b727220a9p+1, 0x1.3f84eafa3ea68p-53, 0x1.bb81b6c52b327p-105},  // e = 8
    {0x1.f306dc9c882a4p+0, 0x1.3f84eafa3ea69p-52, 0x1.77036d8a5664fp-105},  // e = 9
    {0x1.f306dc9c882a5p+1, 0x1.fc2757d1f534cp-54, 0x1.dc0db6295993cp-106},  // e = 10
    {0x1.e60db9391054ap+1, 0x1.fc2757d1f534cp-53, 0x1.dc0db6295993cp-105},  // e = 11
    {0x1.cc1b727220a94p+1, 0x1.fc2757d1f534dp-52, 0x1.b81b6c52b3278p-105},  // e = 12
    {0x1.9836e4e441529p+1, 0x1.f84eafa3ea69bp-52, 0x1.7036d8a5664f1p-105},  // e = 13
    {0x1.306dc9c882a53p+1, 0x1.f09d5f47d4d37p-52, 0x1.c0db6295993c4p-106},  // e = 14
    {0x1.836e4e441529cp-1, 0x1.e13abe8fa9a6ep-52, 0x1.c0db6295993c4p-105},  // e = 15
    {0x1.836e4e441529ep+0, 0x1.c2757d1f534ddp-52, 0x1.81b6c52b32788p-105},  // e = 16
    {0x1.836e4e441529fp+1, 0x1.84eafa3ea69bbp-52, 0x1.036d8a5664f10p-105},  // e = 17
    {0x1.06dc9c882a53fp+1, 0x1.09d5f47d4d377p-52, 0x1.b6c52b3278840p-111},  // e = 18
    {0x1.b727220a94fe0p-4, 0x1.3abe8fa9a6ee0p-56, 0x1.b6c52b3278860p-110},  // e = 19
    {0x1.b727220a94fe0p-3, 0x1.3abe8fa9a6ee0p-55, 0x1.b6c52b3278870p-109},  // e = 20
    {0x1.b727220a94fe0p-2, 0x1.3abe8fa9a6ee0p-54, 0x1.b6c52b3278870p-108},  // e = 21
    {0x1.b727220a94fe0p-1, 0x1.3abe8fa9a6ee0p-53, 0x1.b6c52b3278870p-107},  // e = 22
    {0x1.b727220a94fe0p+0, 0x1.3abe8fa9a6ee0p-52, 0x1.b6c52b3278872p-106},  // e = 23
    {0x1.b727220a94fe1p+1, 0x1.d5f47d4d37700p-54, 0x1.b6c52b3278872p-105},  // e = 24
    {0x1.6e4e441529fc2p+1, 0x1.d5f47d4d37702p-53, 0x1.6d8a5664f10e4p-105},  // e = 25
    {0x1.b9391054a7f08p+0, 0x1.d5f47d4d37703p-52, 0x1.b6295993c4390p-106},  // e = 26
    {0x1.b9391054a7f09p+1, 0x1.abe8fa9a6ee06p-52, 0x1.b6295993c4390p-105},  // e = 27
    {0x1.727220a94fe13p+1, 0x1.57d1f534ddc0dp-52, 0x1.6c52b32788720p-105},  // e = 28
    {0x1.c9c882a53f84ep+0, 0x1.5f47d4d377036p-53, 0x1.b14acc9e21c82p-106},  // e = 29
    {0x1.c9c882a53f84ep+1, 0x1.5f47d4d377036p-52, 0x1.b14acc9e21c82p-105},  // e = 30
    {0x1.9391054a7f09dp+1, 0x1.7d1f534ddc0dap-53, 0x1.6295993c43904p-105},  // e = 31
    {0x1.27220a94fe13ap+1, 0x1.7d1f534ddc0dbp-52, 0x1.8a5664f10e410p-106},  // e = 32
    {0x1.391054a7f09d4p-1, 0x1.f47d4d377036cp-53, 0x1.8a5664f10e410p-105},  // e = 33
    {0x1.391054a7f09d4p+0, 0x1.f47d4d377036dp-52, 0x1.14acc9e21c820p-105},  // e = 34
    {0x1.391054a7f09d5p+1, 0x1.e8fa9a6ee06dbp-52, 0x1.4acc9e21c8208p-108},  // e = 35
    {0x1.c882a53f84eacp-1, 0x1.d1f534ddc0db6p-52, 0x1.4acc9e21c820cp-107},  // e = 36
    {0x1.c882a53f84eaep+0, 0x1.a3ea69bb81b6cp-52, 0x1.4acc9e21c820ep-106},  // e = 37
    {0x1.c882a53f84eafp+1, 0x1.47d4d377036d8p-52, 0x1.4acc9e21c820fp-105},  // e = 38
    {0x1.91054a7f09d5fp+1, 0x1.1f534ddc0db62p-53, 0x1.2b3278872083ep-106},  // e = 39
    {0x1.220a94fe13abep+1, 0x1.1f534ddc0db62p-52, 0x1.2b3278872083fp-105},  // e = 40
    {0x1.1054a7f09d5f4p-1, 0x1.f534ddc0db628p-55, 0x1.5993c439041fcp-107},  // e = 41
    {0x1.1054a7f09d5f4p+0, 0x1.f534ddc0db628p-54, 0x1.5993c439041fep-106},  // e = 42
    {0x1.1054a7f09d5f4p+1, 0x1.f534ddc0db628p-53, 0x1.5993c439041fep-105},  // e = 43
    {0x1.054a7f09d5f40p-2, 0x1.f534ddc0db629p-52, 0x1.664f10e4107f8p-106},  // e = 44
    {0x1.054a7f09d5f44p-1, 0x1.ea69bb81b6c52p-52, 0x1.664f10e4107f9p-105},  // e = 45
    {0x1.054a7f09d5f46p+0, 0x1.d4d377036d8a5p-52, 0x1.993c439041fe4p-106},  // e = 46
    {0x1.054a7f09d5f47p+1, 0x1.a9a6ee06db14ap-52, 0x1.993c439041fe5p-105},  // e = 47
    {0x1.529fc2757d1e0p-4, 0x1.534ddc0db6295p-52, 0x1.3278872083fcap-105},  // e = 48
    {0x1.529fc2757d1f0p-3, 0x1.4d377036d8a56p-53, 0x1.93c439041fe50p-107},  // e = 49
    {0x1.529fc2757d1f0p-2, 0x1.4d377036d8a56p-52, 0x1.93c439041fe50p-106},  // e = 50
    {0x1.529fc2757d1f4p-1, 0x1.34ddc0db62958p-53, 0x1.93c439041fe51p-105},  // e = 51
    {0x1.529fc2757d1f4p+0, 0x1.34ddc0db62959p-52, 0x1.278872083fca2p-105},  // e = 52
    {0x1.529fc2757d1f5p+1, 0x1.a6ee06db14accp-54, 0x1.3c439041fe514p-107},  // e = 53
    {0x1.4a7f09d5f47d4p+0, 0x1.a6ee06db14accp-53, 0x1.3c439041fe516p-106},  // e = 54
    {0x1.4a7f09d5f47d4p+1, 0x1.a6ee06db14accp-52, 0x1.3c439041fe516p-105},  // e = 55
    {0x1.29fc2757d1f52p+0, 0x1.4ddc0db629599p-52, 0x1.e21c820ff28b0p-107},  // e = 56
    {0x1.29fc2757d1f53p+1, 0x1.377036d8a5664p-53, 0x1.e21c820ff28b0p-106},  // e = 57
    {0x1.4fe13abe8fa98p-1, 0x1.377036d8a5664p-52, 0x1.e21c820ff28b1p-105},  // e = 58
    {0x1.4fe13abe8fa9ap+0, 0x1.bb81b6c52b324p-54, 0x1.c439041fe5163p-105},  // e = 59
    {0x1.4fe13abe8fa9ap+1, 0x1.bb81b6c52b326p-53, 0x1.8872083fca2c7p-105},  // e = 60
    {0x1.3f84eafa3ea68p+0, 0x1.bb81b6c52b327p-52, 0x1.10e4107f9458ep-105},  // e = 61
    {0x1.3f84eafa3ea69p+1, 0x1.77036d8a5664fp-52, 0x1.0e4107f9458e8p-108},  // e = 62
    {0x1.fc2757d1f534cp-1, 0x1.dc0db6295993cp-53, 0x1.0e4107f9458e8p-107},  // e = 63
    {0x1.fc2757d1f534cp+0, 0x1.dc0db6295993cp-52, 0x1.0e4107f9458eap-106},  // e = 64
    {0x1.fc2757d1f534dp+1, 0x1.b81b6c52b3278p-52, 0x1.0e4107f9458eap-105},  // e = 65
    {0x1.f84eafa3ea69bp+1, 0x1.7036d8a5664f1p-52, 0x1.c820ff28b1d50p-109},  // e = 66
    {0x1.f09d5f47d4d37p+1, 0x1.c0db6295993c4p-53, 0x1.c820ff28b1d58p-108},  // e = 67
    {0x1.e13abe8fa9a6ep+1, 0x1.c0db6295993c4p-52, 0x1.c820ff28b1d5cp-107},  // e = 68
    {0x1.c2757d1f534ddp+1, 0x1.81b6c52b32788p-52, 0x1.c820ff28b1d5ep-106},  // e = 69
    {0x1.84eafa3ea69bbp+1, 0x1.036d8a5664f10p-52, 0x1.c820ff28b1d5ep-105},  // e = 70
    {0x1.09d5f47d4d377p+1, 0x1.b6c52b3278840p-58, 0x1.9041fe5163abdp-105},  // e = 71
    {0x1.3abe8fa9a6ee0p-3, 0x1.b6c52b3278860p-57, 0x1.2083fca2c757bp-105},  // e = 72
    {0x1.3abe8fa9a6ee0p-2, 0x1.b6c52b3278870p-56, 0x1.041fe5163abdcp-107},  // e = 73
    {0x1.3abe8fa9a6ee0p-1, 0x1.b6c52b3278870p-55, 0x1.041fe5163abdep-106},  // e = 74
    {0x1.3abe8fa9a6ee0p+0, 0x1.b6c52b3278870p-54, 0x1.041fe5163abdep-105},  // e = 75
    {0x1.3abe8fa9a6ee0p+1, 0x1.b6c52b3278872p-53, 0x1.07f9458eaf7a0p-110},  // e = 76
    {0x1.d5f47d4d37700p-1, 0x1.b6c52b3278872p-52, 0x1.07f9458eaf7a0p-109},  // e = 77
    {0x1.d5f47d4d37702p+0, 0x1.6d8a5664f10e4p-52, 0x1.07f9458eaf7a8p-108},  // e = 78
    {0x1.d5f47d4d37703p+1, 0x1.b6295993c4390p-53, 0x1.07f9458eaf7acp-107},  // e = 79
    {0x1.abe8fa9a6ee06p+1, 0x1.b6295993c4390p-52, 0x1.07f9458eaf7aep-106},  // e = 80
    {0x1.57d1f534ddc0dp+1, 0x1.6c52b32788720p-52, 0x1.07f9458eaf7aep-105},  // e = 81
    {0x1.5f47d4d377036p+0, 0x1.b14acc9e21c82p-53, 0x1.fe5163abdeba0p-110},  // e = 82
    {0x1.5f47d4d377036p+1, 0x1.b14acc9e21c82p-52, 0x1.fe5163abdebb0p-109},  // e = 83
    {0x1.7d1f534ddc0dap+0, 0x1.6295993c43904p-52, 0x1.fe5163abdebb8p-108},  // e = 84
    {0x1.7d1f534ddc0dbp+1, 0x1.8a5664f10e410p-53, 0x1.fe5163abdebbcp-107},  // e = 85
    {0x1.f47d4d377036cp+0, 0x1.8a5664f10e410p-52, 0x1.fe5163abdebbcp-106},  // e = 86
    {0x1.f47d4d377036dp+1, 0x1.14acc9e21c820p-52, 0x1.fe5163abdebbcp-105},  // e = 87
    {0x1.e8fa9a6ee06dbp+1, 0x1.4acc9e21c8208p-55, 0x1.fca2c757bd778p-105},  // e = 88
    {0x1.d1f534ddc0db6p+1, 0x1.4acc9e21c820cp-54, 0x1.f9458eaf7aef1p-105},  // e = 89
    {0x1.a3ea69bb81b6cp+1, 0x1.4acc9e21c820ep-53, 0x1.f28b1d5ef5de2p-105},  // e = 90
    {0x1.47d4d377036d8p+1, 0x1.4acc9e21c820fp-52, 0x1.e5163abdebbc5p-105},  // e = 91
    {0x1.1f534ddc0db62p+0, 0x1.2b3278872083ep-53, 0x1.ca2c757bd778ap-105},  // e = 92
    {0x1.1f534ddc0db62p+1, 0x1.2b3278872083fp-52, 0x1.9458eaf7aef15p-105},  // e = 93
    {0x1.f534ddc0db628p-2, 0x1.5993c439041fcp-54, 0x1.28b1d5ef5de2bp-105},  // e = 94
    {0x1.f534ddc0db628p-1, 0x1.5993c439041fep-53, 0x1.458eaf7aef158p-107},  // e = 95
    {0x1.f534ddc0db628p+0, 0x1.5993c439041fep-52, 0x1.458eaf7aef158p-106},  // e = 96
    {0x1.f534ddc0db629p+1, 0x1.664f10e4107f8p-53, 0x1.458eaf7aef158p-105},  // e = 97
    {0x1.ea69bb81b6c52p+1, 0x1.664f10e4107f9p-52, 0x1.163abdebbc560p-106},  // e = 98
    {0x1.d4d377036d8a5p+1, 0x1.993c439041fe4p-53, 0x1.163abdebbc561p-105},  // e = 99
    {0x1.a9a6ee06db14ap+1, 0x1.993c439041fe5p-52, 0x1.63abdebbc5618p-108},  // e = 100
    {0x1.534ddc0db6295p+1, 0x1.3278872083fcap-52, 0x1.63abdebbc5618p-107},  // e = 101
    {0x1.4d377036d8a56p+0, 0x1.93c439041fe50p-54, 0x1.63abdebbc561ap-106},  // e = 102
    {0x1.4d377036d8a56p+1, 0x1.93c439041fe50p-53, 0x1.63abdebbc561bp-105},  // e = 103
    {0x1.34ddc0db62958p+0, 0x1.93c439041fe51p-52, 0x1.8eaf7aef1586cp-106},  // e = 104
};

// sin/cos of any fp32 angle in fp64: the Cody-Waite form up to 2^24, the
// Payne-Hanek reduction (see the file header) above it, one polynomial
// evaluation for both; inf and NaN give NaN.
MI_SINCOS_HD inline void rope_sincos_any(float a, double* s_out, double* c_out) {
    const float fa = fabsf(a);
    double r;
    int q;
    if (fa <= 16777216.0f) {
        const double kQ1 = 0x1.921fb54p+0, kQ2 = 0x1.10b46p-30, kQ3 = 0x1.1a62633145c07p-54;
        const double ad = static_cast<double>(a);
        const double k = rint(ad * 0x1.45f306dc9c883p-1);
        r = fma(-k, kQ3, fma(-k, kQ2, fma(-k, kQ1, ad)));
        q = static_cast<int>(static_cast<long long>(k) & 3);
    } else if (fa <= 3.4028234663852886e38f) {
        uint32_t bits;
        memcpy(&bits, &fa, 4);
        const int e = static_cast<int>(bits >> 23) - 150;             // 1 .. 104
        const double m = static_cast<double>((bits & 0x7fffffu) | 0x800000u);
        const double* y = kTwoOverPiMod4[e - 1];
        const double p0 = m * y[0];
        const double e0 = fma(m, y[0], -p0);                          // exact
        const double hi = p0 - 4.0 * floor(p0 * 0.25);                // exact, in [0, 4)
        const double lo = e0 + fma(m, y[1], m * y[2]);               // |lo| < 2^-26
        const double k = rint(hi + lo);
        const double f = (hi - k) + lo;                               // hi - k exact
        r = fma(f, 0x1.921fb54442d18p+0, f * 0x1.1a62633145c07p-54);  // f * pi/2
        q = static_cast<int>(k) & 3;
        if (a < 0.0f) q = (4 - q) & 3, r = -r;  // sin odd, cos even: reduce -a
    } else {  // inf, NaN
        *s_out = *c_out = static_cast<double>(fa - fa);
        return;
    }
    rope_sincos_quadrant(r, q, s_out, c_out);
    if (a == 0.0f) *s_out = static_cast<double>(a);  // sin(-0) = -0
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
