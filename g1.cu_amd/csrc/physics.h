// physics.h -- one G1 physics substep for one world on a 32-lane group (gfx950 / CDNA4).
//
// Mapping (two worlds per wave64, see lanes.h):
//   * tree sweeps (FK, RNE velocity/acceleration, RNE force gather, articulated-inertia
//     downdate): lane l == body l (0 = world, 1 = pelvis/free joint, 2..30 hinges, 31 idle).
//     Sweeps run level-synchronously over tree depth; a parent gathers its children's
//     contributions in descending child index, exactly the order of the reference's serial
//     leaf->root loops, so every accumulated value has the reference's rounding sequence.
//     The smooth solve (M+dtB)^-1(tau-bias) rides on the factor's leaf->root sweep and a
//     level-synchronous root->leaf sweep.
//   * contact M^-1 solves: lane j == right-hand side j (1+3c+a: contact basis e_{c,a}); the tree
//     traversal is fully unrolled over the static topology so the per-column articulated bias
//     forces stay in registers; the shared factor is read from LDS (same address on all lanes =
//     broadcast).
//   * contact rows: lane i == constraint row i (4 per contact); lane i holds column i of A
//     (== row i, A is symmetric bit-for-bit) in registers for the projected Gauss-Seidel sweeps.
//
// Reference algorithm (Infatoshi/g1.cu): FK src/dynamics.cuh:47-88; motion axes + RNE bias
// src/aba_bias.cuh:17-121; damped ABA factor src/aba_factor.cuh:44-109; M^-1 apply
// src/aba_factor.cuh:121-165; foot contact + 3-basis Gram + PGS src/env_qacc.cuh:52-211,
// src/contact.cuh:31-57,97-109,159-171; Euler + quaternion integration src/dynamics.cuh:333-355,
// src/g1_env.cu:154-162.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "g1_model_tables.h"
#include "lanes.h"
#include "tree.h"

namespace g1k {

using namespace g1;
using MF = ModelT<float>;

constexpr int kCols = 1 + 3 * kNFoot;  // smooth column + 3 basis columns per contact
constexpr int kChainSolveCon = 2;      // contacts per world up to which the M^-1 solves use the chain layout
constexpr int kMmStride = 37;          // odd stride: column-parallel LDS reads are conflict-free
constexpr int kRow = 8;              // row stride of the motion axes S and factor rows U (6 + 2 used):
                                     // 16-byte rows, read whole by 16-byte LDS instructions
constexpr int kInvD = 6, kUs = 7;    // columns of a hinge factor row past I^A S
constexpr int kPairs = kNFoot * (kNFoot + 1) / 2;

struct V3 { float x, y, z; };
struct Q4 { float w, x, y, z; };

// Fused multiply-add is used only explicitly (the build passes -ffp-contract=off), with one
// convention shared with the CPU restatement: a sum of products a0 b0 + a1 b1 + ... is evaluated
// left to right as s = a0 b0, s = fma(a_i, b_i, s) (differences as fma(-a_i, b_i, s)); an
// accumulation s = 0; s += a_i b_i as s = fma(a_i, b_i, s) from s = 0; x + a b as fma(a, b, x).
__device__ __forceinline__ float fmaf_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

__device__ __forceinline__ V3 vadd(V3 a, V3 b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
__device__ __forceinline__ V3 vsub(V3 a, V3 b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
__device__ __forceinline__ V3 cross(V3 a, V3 b) {
  return {fmaf_(-a.z, b.y, a.y * b.z), fmaf_(-a.x, b.z, a.z * b.x), fmaf_(-a.y, b.x, a.x * b.y)};
}
__device__ __forceinline__ float dot3(V3 a, V3 b) { return fmaf_(a.z, b.z, fmaf_(a.y, b.y, a.x * b.x)); }
__device__ __forceinline__ Q4 qmul(Q4 a, Q4 b) {
  return {fmaf_(-a.z, b.z, fmaf_(-a.y, b.y, fmaf_(-a.x, b.x, a.w * b.w))),
          fmaf_(-a.z, b.y, fmaf_(a.y, b.z, fmaf_(a.x, b.w, a.w * b.x))),
          fmaf_(a.z, b.x, fmaf_(a.y, b.w, fmaf_(-a.x, b.z, a.w * b.y))),
          fmaf_(a.z, b.w, fmaf_(-a.y, b.x, fmaf_(a.x, b.y, a.w * b.z)))};
}
// v' = v + w t + u x t, t = 2 u x v
__device__ __forceinline__ V3 qrot(Q4 q, V3 v) {
  const V3 u{q.x, q.y, q.z};
  const V3 c = cross(u, v);
  const V3 t{2.f * c.x, 2.f * c.y, 2.f * c.z};
  const V3 ut = cross(u, t);
  return {fmaf_(q.w, t.x, v.x) + ut.x, fmaf_(q.w, t.y, v.y) + ut.y, fmaf_(q.w, t.z, v.z) + ut.z};
}
// fp64 forms of the above for the forward-kinematics compositions (same operation order; qrotd the
// same values)
struct V3d { double x, y, z; };
struct Q4d { double w, x, y, z; };
__device__ __forceinline__ double fmad_(double a, double b, double c) { return __builtin_fma(a, b, c); }
__device__ __forceinline__ V3d vaddd(V3d a, V3d b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
__device__ __forceinline__ V3d crossd(V3d a, V3d b) {
  return {fmad_(-a.z, b.y, a.y * b.z), fmad_(-a.x, b.z, a.z * b.x), fmad_(-a.y, b.x, a.x * b.y)};
}
__device__ __forceinline__ Q4d qmuld(Q4d a, Q4d b) {
  return {fmad_(-a.z, b.z, fmad_(-a.y, b.y, fmad_(-a.x, b.x, a.w * b.w))),
          fmad_(-a.z, b.y, fmad_(a.y, b.z, fmad_(a.x, b.w, a.w * b.x))),
          fmad_(a.z, b.x, fmad_(a.y, b.w, fmad_(-a.x, b.z, a.w * b.y))),
          fmad_(a.z, b.w, fmad_(-a.y, b.x, fmad_(a.x, b.y, a.w * b.z)))};
}
// The same values as qrot's sequence in fp64, in two fewer operations: with c = u x v, t = 2c and
// u x t = 2 (u x c) are exact doublings (the operands are fp32 values and products of them, far from
// fp64's underflow), so fma(w, t, v) + u x t = fma(2, u x c, fma(2w, c, v)) bit for bit.
__device__ __forceinline__ V3d qrotd(Q4d q, V3d v) {
  const V3d u{q.x, q.y, q.z};
  const V3d c = crossd(u, v);
  const V3d X = crossd(u, c);
  const double w2 = q.w + q.w;
  return {fmad_(2.0, X.x, fmad_(w2, c.x, v.x)), fmad_(2.0, X.y, fmad_(w2, c.y, v.y)),
          fmad_(2.0, X.z, fmad_(w2, c.z, v.z))};
}
__device__ __forceinline__ double gshfld(double v, int src) { return __shfl(v, src, kGroup); }

// Correctly rounded fp32 transcendentals (evaluated in fp64, rounded once; fp64 VALU issues like
// fp32, at about twice its VALU time, and these sit outside the inner loops). The contact force is stiff in the
// foot height, so a 1-ulp difference in an FK rotation moves qacc by up to ~1e-4 relative on
// shallow penetrations; correct rounding makes every transcendental reproducible bit-for-bit.
__device__ __forceinline__ float sin_rn(float x) { return (float)sin((double)x); }
__device__ __forceinline__ float cos_rn(float x) { return (float)cos((double)x); }
// both from one fp64 argument reduction
__device__ __forceinline__ void sincos_rn(float x, float& sn, float& cs) {
  double sd, cd;
  sincos((double)x, &sd, &cd);
  sn = (float)sd;
  cs = (float)cd;
}

// One Horner step fma(z, p, c) as the three-address v_fma_f64. The coefficients below stay in
// vector registers across the substep loop, and for fma(z, p, c) the compiler otherwise copies c
// into the accumulator (v_mov_b64) for the two-address v_fmac_f64: one VALU instruction per step
// fewer, the same operation.
__device__ __forceinline__ double horner_d(double z, double p, double c) {
  double r;
  __asm__("v_fma_f64 %0, %1, %2, %3" : "=v"(r) : "v"(z), "v"(p), "v"(c));
  return r;
}
// sin_rn and cos_rn of one argument for the hinge half-angles on a short fp64 path for |x| <= 4:
// k = rint(x 2/pi), r = (x - k P1) - k P2 with P1 + P2 = pi/2 (P1 = RN(pi/2), so x - k P1 is exact
// in the fma: both are multiples of 2^-52 and the difference is below 1), the Taylor series of
// sin to r^15 and cos to r^14 by Horner (truncation at |r| = pi/4: 5e-17 and 1e-15 absolute), the
// quadrant k mod 4 by selects and one rounding to float. For every float with |x| <= 4 this
// equals the fp64-libm value rounded to float (tests: the probe g1_probe_sincos_hinge against the
// oracle over all of them; one term fewer in either series breaks it for a few dozen), so the
// 24-bit rounding absorbs the truncation; larger or non-finite x take the library. The two terms
// that a series with margin would add cost the kernel its second wave per SIMD (their constants
// are held in vector registers across the substep loop).
__device__ __forceinline__ void sincos_hinge_rn(float x, float& sn, float& cs) {
  if (fabsf(x) <= 4.f) {
    const double xd = x;
    const double kd = __builtin_rint(xd * 0.63661977236758134308);
    const double r = __builtin_fma(-kd, 6.123233995736766e-17, __builtin_fma(-kd, 1.5707963267948966, xd));
    const double z = r * r;
    double ps = -1.0 / 1307674368000.0;
    ps = horner_d(z, ps, 1.0 / 6227020800.0);
    ps = horner_d(z, ps, -1.0 / 39916800.0);
    ps = horner_d(z, ps, 1.0 / 362880.0);
    ps = horner_d(z, ps, -1.0 / 5040.0);
    ps = horner_d(z, ps, 1.0 / 120.0);
    ps = horner_d(z, ps, -1.0 / 6.0);
    double pc = -1.0 / 87178291200.0;
    pc = horner_d(z, pc, 1.0 / 479001600.0);
    pc = horner_d(z, pc, -1.0 / 3628800.0);
    pc = horner_d(z, pc, 1.0 / 40320.0);
    pc = horner_d(z, pc, -1.0 / 720.0);
    pc = horner_d(z, pc, 1.0 / 24.0);
    pc = __builtin_fma(z, pc, -0.5);
    const double sr = __builtin_fma(r * z, ps, r), cr = __builtin_fma(z, pc, 1.0);
    // (sin x, cos x) = (sin r, cos r), (cos r, -sin r), (-sin r, -cos r), (-cos r, sin r) for k mod 4
    const int k = (int)kd;
    const float so = (float)((k & 1) ? cr : sr), co = (float)((k & 1) ? sr : cr);
    sn = (k & 2) ? -so : so;
    cs = ((k + 1) & 2) ? -co : co;
    if (x == 0.f) sn = x;   // sin(-0) = -0 (r = +0 there)
  } else {
    sincos_rn(x, sn, cs);
  }
}

// sin_rn and cos_rn of one argument on a short path for |x| <= 1/8 (the free joint's half rotation
// per substep): the fp64 Taylor series by Horner, sin to x^11 and cos to x^12 (truncation below
// 2^-68 relative), coefficients (-1)^k / n! rounded once, then one rounding to float. For every
// float with |x| <= 1/8 this equals the fp64-libm value rounded to float (tests: the probe
// g1_probe_sincos against the oracle over all of them); larger or non-finite x take the library.
__device__ __forceinline__ void sincos_small_rn(float x, float& sn, float& cs) {
  if (fabsf(x) <= 0.125f) {
    const double xd = x, z = xd * xd;
    double ps = -1.0 / 39916800.0;
    ps = horner_d(z, ps, 1.0 / 362880.0);
    ps = horner_d(z, ps, -1.0 / 5040.0);
    ps = horner_d(z, ps, 1.0 / 120.0);
    ps = horner_d(z, ps, -1.0 / 6.0);
    double pc = 1.0 / 479001600.0;
    pc = horner_d(z, pc, -1.0 / 3628800.0);
    pc = horner_d(z, pc, 1.0 / 40320.0);
    pc = horner_d(z, pc, -1.0 / 720.0);
    pc = horner_d(z, pc, 1.0 / 24.0);
    pc = __builtin_fma(z, pc, -0.5);
    const float s_ = (float)__builtin_fma(xd * z, ps, xd);
    sn = (x == 0.f) ? x : s_;   // sin(-0) = -0
    cs = (float)__builtin_fma(z, pc, 1.0);
  } else {
    sincos_hinge_rn(x, sn, cs);
  }
}

// Correctly rounded reciprocal and quotient on short dependency chains, for the positive normal
// divisors of this path (pivots, D = S'I^A S + armature + dt kd, A_ii, impedances, angles).
// rcp_rn: one Newton step y = y0 + y0 (1 - b y0) (fused) on the hardware estimate y0 returns
// RN(1/b); checked bit-exact against the IEEE division for every mantissa of the binades
// 2^-30 .. 2^30. div_rn: with y = RN(1/b), q0 = RN(a y), the residual a - b q0 is exact in an
// fma and RN(q0 + r y) = RN(a / b) (Markstein's theorem); also checked bit-exact against the
// IEEE division on 2e9 operand pairs. Both replace the ~10-instruction scaled IEEE sequence.
__device__ __forceinline__ float rcp_rn(float b) {
  const float y0 = __builtin_amdgcn_rcpf(b);
  return __builtin_fmaf(__builtin_fmaf(-b, y0, 1.f), y0, y0);
}
__device__ __forceinline__ float div_rn(float a, float b, float yb) {
  const float q0 = a * yb;
  return __builtin_fmaf(__builtin_fmaf(-q0, b, a), yb, q0);
}
// div_rn for numerators that may be infinite (the observation's normalisation: a state set from
// outside can hold +-inf velocities): the residual of an infinite q0 is NaN, so q0 itself is
// returned there, which is the IEEE quotient +-inf for an infinite numerator (and, within an ulp
// of overflow, the same +-inf or FLT_MAX that any later clamp maps alike).
__device__ __forceinline__ float div_rn_inf(float a, float b, float yb) {
  const float q0 = a * yb;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, b, a), yb, q0);
  return __builtin_isinf(q0) ? q0 : q;
}
__device__ __forceinline__ float rsqrt_rn(float x) { return rcp_rn(sqrtf(x)); }
// Correctly rounded square root of x >= 2^-96 (and of +0, +inf): the hardware root s is within
// one ulp, and the residuals x - s_dn s and x - s_up s of its neighbours select RN(sqrt x). The
// compiler's sqrtf makes the same selection after scaling arguments below 2^-96 and routing 0,
// inf and NaN around it; the Cholesky pivots (Schur complements of the free joint's articulated
// inertia, of the order of the robot's mass and inertia) need neither. Checked bit-exact against
// the IEEE square root for every float from 2^-96 up, +0 and +inf.
__device__ __forceinline__ float sqrt_rn_pos(float x) {
  const float s = __builtin_amdgcn_sqrtf(x);
  const float sd = __int_as_float(__float_as_int(s) - 1), su = __int_as_float(__float_as_int(s) + 1);
  const float r = __builtin_fmaf(-sd, s, x) <= 0.f ? sd : s;
  return __builtin_fmaf(-su, s, x) > 0.f ? su : r;
}

__device__ __forceinline__ Q4 qnorm(Q4 q) {
  float n = rsqrt_rn(fmaf_(q.z, q.z, fmaf_(q.y, q.y, fmaf_(q.x, q.x, q.w * q.w))));
  return {q.w * n, q.x * n, q.y * n, q.z * n};
}
struct M3 { float m[9]; };
__device__ __forceinline__ M3 quat2mat(Q4 q) {
  float w = q.w, x = q.x, y = q.y, z = q.z;
  M3 r;
  // 1 - 2 s is fma(-2, s, 1) exactly (2 s is exact)
  r.m[0] = fmaf_(-2.f, fmaf_(z, z, y * y), 1.f); r.m[1] = 2.f * fmaf_(-w, z, x * y); r.m[2] = 2.f * fmaf_(w, y, x * z);
  r.m[3] = 2.f * fmaf_(w, z, x * y); r.m[4] = fmaf_(-2.f, fmaf_(z, z, x * x), 1.f); r.m[5] = 2.f * fmaf_(-w, x, y * z);
  r.m[6] = 2.f * fmaf_(-w, y, x * z); r.m[7] = 2.f * fmaf_(w, x, y * z); r.m[8] = fmaf_(-2.f, fmaf_(y, y, x * x), 1.f);
  return r;
}
__device__ __forceinline__ void crossm(V3 w1, V3 v1, V3 w2, V3 v2, V3& ow, V3& ov) {
  ow = cross(w1, w2);
  V3 a = cross(w1, v2), b = cross(v1, w2);
  ov = {a.x + b.x, a.y + b.y, a.z + b.z};
}

__device__ __forceinline__ int symidx(int i, int j) {
  if (i > j) { int t = i; i = j; j = t; }
  return i * 6 - (i * (i - 1)) / 2 + (j - i);
}
// The free joint's motion subspace S_base: translation k = (0,0,0, e_k), rotation k = (R1 col k,
// 0,0,0). Its products below skip the structural zeros (a generic 6-term sum adds exact zeros to
// the one or three nonzero terms in the same order), which can change only the sign of an
// exactly-zero result: -0 and +0 compare equal, and no later operation distinguishes them (every
// divisor is positive). The oracle keeps the generic products.
// S_base row k . x for k = 0..5 (x a 6-vector; R1col[k] = column k of R1 in S rows 3..5)
__device__ __forceinline__ float sbase_dot(int k, const float* Srow, const float* x) {
  return k < 3 ? x[3 + k] : fmaf_(Srow[2], x[2], fmaf_(Srow[1], x[1], Srow[0] * x[0]));
}
// component i of S_base' q (q the 6 base dofs): angular rows from the rotations, linear from the
// translations
__device__ __forceinline__ float sbase_col(int i, const float (&S3)[3][3], const float* q) {
  return i < 3 ? fmaf_(S3[2][i], q[5], fmaf_(S3[1][i], q[4], S3[0][i] * q[3])) : q[i - 3];
}

__device__ __forceinline__ float dot6(const float* a, const float* b) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 6; ++i) s = fmaf_(a[i], b[i], s);
  return s;
}

// Scheduling pin for the unrolled tree traversals: forces the six carried values through a
// (no-op) volatile asm, which no LDS access crosses. Without it the unrolled code hoists every
// body's loads up front and runs out of registers; the traversals issue the next body's reads
// before the pin, so one body's reads are in flight while the current body computes.
#define G1_PIN6(v) __asm__ volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5])::"memory")

// MuJoCo solimp impedance sigmoid (reference: src/contact.cuh:97-109)
__device__ __forceinline__ float foot_impedance(float pos) {
  const float dmin = MF::foot_solimp[0], dmax = MF::foot_solimp[1], width = MF::foot_solimp[2];
  const float mid = MF::foot_solimp[3], power = MF::foot_solimp[4];
  constexpr float inv_width = 1.f / MF::foot_solimp[2];   // RN(1/width), folded at compile time
  float x = div_rn(fabsf(pos), width, inv_width);
  float y;
  if (x >= 1.f) y = 1.f;
  else {
    // The model's solimp power is 2: x^2 of a float is exact in fp64, so the correctly rounded
    // pow(x, 2) is the fp32 product x*x, and mid^(power-1) = mid.
    static_assert(MF::foot_solimp[4] == 2.f, "impedance power 2 assumed");
    float a = 1.f / mid;
    float b = 1.f / (1.f - mid);
    y = (x < mid) ? a * (x * x) : fmaf_(-b, (1.f - x) * (1.f - x), 1.f);
  }
  return fmaf_(y, dmax - dmin, dmin);
}

// ---------------------------------------------------------------- per-world LDS
// Every array starts on a 16-byte boundary: adjacent float reads and writes then combine into
// 8- and 16-byte LDS instructions, which take 16-bit immediate offsets from the world's base
// address; two 4-byte ones combined into a read2/write2 take 8-bit offsets (in words, at most 1020
// bytes), and past that each pair got an address of its own (a vector add per pair).
struct WorldLds {
  union {
    struct {
      alignas(16) float S[kNV][kRow];      // motion axes (world axes about the pelvis origin)
      // hinge factor rows: I^A S (0..5), 1/(S'I^A S + armature + dt kd) (kInvD), the smooth
      // solve's bias u = x - S.pA (kUs); one row is read whole by two 16-byte reads
      alignas(16) float U[kNBody][kRow];
      alignas(16) float Dfac[36];       // Cholesky factor of the free-joint 6x6 block
      alignas(16) float Dinv[6];        // RN(1 / diagonal of Dfac)
      alignas(16) float Dm[36];         // free-joint 6x6 block before factoring
    } fac;
    alignas(16) float G[kPairs][9];     // 3x3 Gram blocks of contact pairs c <= c' (after the solves)
  } u;
  alignas(16) float qvel[kNV + 1];
  union {
    struct {
      alignas(16) float Mm[kCols][kMmStride];          // solve outputs: column 0 = qacc_smooth, 1+3c+a = M^-1 e_{c,a}
      alignas(16) float Eb[kNFoot][3][kContactDofs];   // contact basis rows over the contact's 12 ancestor dofs
    };
    // body spatial inertias as full 6x6 rows (row r of body b: six floats at I6r[b][r]), from the
    // body-inertia phase to the end of the factor, before the solves write Mm and PASS 1 Eb
    alignas(16) float I6r[kNBody][6][6];
  };
  alignas(16) float con[kNFoot][4];                // contact point x, y, z (= pen/2), penetration
  alignas(16) float con_w0[kNFoot];                // invweight0 of the foot body
  alignas(16) int con_leg[kNFoot];                 // 0: left foot (body 7), 1: right foot (body 13)
  alignas(16) float bvec[kMaxEfc];
  alignas(16) float aref[kMaxEfc];
  alignas(16) float Rc[kNFoot];
  alignas(16) float f[kMaxEfc];
  alignas(16) float qacc[kNV + 1];
};

// ---------------------------------------------------------------- per-lane model constants
struct LaneModel {
  int l, b, par, depth, c0, c1, c2, nchild;
  bool body, hinge;
  V3 bpos, ipos, axis, inert;
  Q4 bquat, iquat;
  float mass;
  // actuator of hinge lanes (actuator index b - 2, dof b + 4, qpos b + 5)
  float kp, kd, clo, chi, flo, fhi, qstand, bdt, arm;
};

// The model constants world_qacc reads on every call, as one row per lane of a world group (the
// values lane_model gives the lane: body 0's where the lane has no body, actuator 0's where it has
// no hinge) plus the lane's FK ancestor word and foot sphere: one table base and immediate offsets
// for every field, where a table per field took a base of its own (three scalar instructions) and a
// 64-bit lane address each, every substep.
struct alignas(16) LaneRow {
  float bpos[3], bquat[4], ipos[3], iquat[4], inert[3], axis[3];
  float mass, bdt;              // body mass; dt k_d of the lane's actuator
  unsigned anc;                 // ancestor lanes of the FK rounds, one byte per round (tree.h)
  float foot_lp[3], foot_w0;    // the lane's foot sphere (sphere 0 on lanes >= kNFoot)
  float pad;
};
static_assert(sizeof(LaneRow) == 112, "seven 16-byte loads per row");
struct LaneRows {
  LaneRow r[kGroup];
};
constexpr LaneRows make_lane_rows() {
  LaneRows t{};
  for (int l = 0; l < kGroup; ++l) {
    LaneRow& x = t.r[l];
    const bool body = l >= 1 && l < kNBody, hinge = l >= 2 && l < kNBody;
    const int b = body ? l : 0, j = body ? b - 1 : 0, i = hinge ? b - 2 : 0;
    for (int k = 0; k < 3; ++k) {
      x.bpos[k] = MF::body_pos[3 * b + k];
      x.ipos[k] = MF::body_ipos[3 * b + k];
      x.inert[k] = MF::body_inertia[3 * b + k];
      x.axis[k] = MF::jnt_axis[3 * j + k];
    }
    for (int k = 0; k < 4; ++k) {
      x.bquat[k] = MF::body_quat[4 * b + k];
      x.iquat[k] = MF::body_iquat[4 * b + k];
    }
    x.mass = MF::body_mass[b];
    x.bdt = MF::dt * MF::act_kd[i];   // the single fp32 product lane_model forms
    x.anc = kAncestorWords.w[l];
    const int sph = l < kNFoot ? l : 0;
    for (int k = 0; k < 3; ++k) x.foot_lp[k] = MF::foot_lpos[3 * sph + k];
    x.foot_w0 = MF::foot_invweight0[sph];
    x.pad = 0.f;
  }
  return t;
}
constexpr LaneRows kLaneRows = make_lane_rows();

// Row l from one address (16-byte loads of the used words): the table base goes through an opaque copy (with
// the address visible the compiler folds field offsets into the base's relocation and gives each
// group of fields a base and a 64-bit lane address of its own) and the lane index is unsigned (a
// 32-bit row offset).
__device__ __forceinline__ LaneRow lane_row(int l) {
  static_assert(sizeof(LaneRow) % 16 == 0, "whole 16-byte words per row");
  typedef const __attribute__((address_space(1))) char* GlobalBytes;   // global loads, not flat ones
  typedef const __attribute__((address_space(1))) float* GlobalFloats;
  GlobalBytes base = (GlobalBytes)(reinterpret_cast<const char*>(&kLaneRows.r[0]));
  __asm__("" : "+s"(base));
  GlobalFloats p = (GlobalFloats)(base + (unsigned)l * sizeof(LaneRow));
  float w[sizeof(LaneRow) / 4];
#pragma unroll
  for (int k = 0; k < (int)(sizeof(LaneRow) / 4); ++k) w[k] = p[k];
  LaneRow R;
  __builtin_memcpy(&R, w, sizeof(LaneRow));
  return R;
}

__device__ __forceinline__ LaneModel lane_model(int l) {
  LaneModel L;
  const LaneRow R = lane_row(l);
  L.l = l;
  L.body = (l >= 1 && l < kNBody);
  L.hinge = (l >= 2 && l < kNBody);
  const int b = L.body ? l : 0;
  L.b = b;
  L.par = L.body ? body_parent[b] : l;
  L.depth = L.body ? body_depth[b] : 0;
  L.nchild = L.body ? body_nchild[b] : 0;
  int c0 = body_child[3 * b], c1 = body_child[3 * b + 1], c2 = body_child[3 * b + 2];
  L.c0 = (L.nchild > 0) ? c0 : l;
  L.c1 = (L.nchild > 1) ? c1 : l;
  L.c2 = (L.nchild > 2) ? c2 : l;
  L.bpos = {R.bpos[0], R.bpos[1], R.bpos[2]};
  L.bquat = {R.bquat[0], R.bquat[1], R.bquat[2], R.bquat[3]};
  L.ipos = {R.ipos[0], R.ipos[1], R.ipos[2]};
  L.iquat = {R.iquat[0], R.iquat[1], R.iquat[2], R.iquat[3]};
  L.inert = {R.inert[0], R.inert[1], R.inert[2]};
  L.mass = R.mass;
  L.axis = {R.axis[0], R.axis[1], R.axis[2]};   // one joint per moving body (generator-checked)
  const int i = L.hinge ? b - 2 : 0;
  L.kp = MF::act_kp[i]; L.kd = MF::act_kd[i];
  L.clo = MF::act_ctrl_lo[i]; L.chi = MF::act_ctrl_hi[i];
  L.flo = MF::act_frc_lo[i]; L.fhi = MF::act_frc_hi[i];
  L.qstand = L.hinge ? MF::qpos_stand[b + 5] : 0.f;
  L.bdt = R.bdt;
  L.arm = L.hinge ? MF::dof_armature[b + 4] : 0.f;
  return L;
}

// ---------------------------------------------------------------- per-lane world state
// Every lane carries the free joint (qpos[0:7], qvel[0:6]; lane 1 is its lane in the tree and the
// one that stores it); hinge lane b carries qpos[b+5], qvel[b+4] and actuator b-2 (PD target,
// previous and current action).
struct LaneState {
  float bq[7], bqd[6];
  float jq, jqd;
};

struct SolveParams {
  int pgs;
  float mu;
  bool damped;   // fold dt*kd into the factor (the env's implicit PD); false = plain M^-1
  bool contact;  // foot-ground contact on/off
};

// One projected Gauss-Seidel sweep over rows II.. (reference: src/contact.cuh:159-171), in the
// row-scaled residual form: row i is held scaled by y_i = RN(1/A_ii) with its diagonal entry 0
// (a_ij = RN(A_ij y_i); A is symmetric bit for bit, so lane i's column of A is its row) together
// with its residual r_i = c_i + sum_j a_ij f_j for the current f, c_i = RN(b_i y_i). Row ii: its
// lane sets f_ii = max(0, -r_ii); the change d = RN(f new - f old) goes from that lane to every
// lane of the world, and every row j adds a_j,ii d to r_j in one fma. Every lane evaluates the
// update and only row ii's lanes keep it; a row past its world's count holds zero entries,
// r = c = 0 and f = 0. Straight-line rows; rows come four to a contact (the wave's largest row
// count nefc_max is a multiple of 4), so the sweep tests nefc_max at every fourth row and branches
// once to its end. W: the rows a world can hold in this wave (nefc_max <= W): lane i holds row i
// and the change is broadcast over its first 16-lane row (16) or its quad (4); for W = 32 see
// pgs_row_pair.
//
// A row in VALU code (W = 16): fn = max(-r, 0), d = fn - f, f = fn on row II's lanes (a lane
// mask), then r += a d with d taken from lane II of the 16-lane row by DPP row_newbcast inside the
// fma (v_fmac_f32 with a DPP source operand): 4 VALU. Written out because the compiler keeps the
// DPP move apart from an fma (it forms the two-operand v_fmac_f32 only after its DPP combining)
// and, with the fma written out alone, adds a canonicalising max before max(-r, 0); these are the
// compiler's own instructions for the operations, so the values are the same. The s_nop and the
// v_cndmask before the DPP read give the two wait states it needs after the VALU write of its
// source. max(-r, 0) is 0 for a NaN r (the quiet NaNs of arithmetic), as t > 0 ? t : 0 is.
// `lanes`: the row's lanes, lane II of every 16-lane row (a mask built from an opaque base in each
// sweep: as 32 constants the compiler holds the masks in scalar registers across the sweep loop
// and spills them).
template <int II, int W>
__device__ __forceinline__ void pgs_row(float a, int l, unsigned long long lanes, float& fi, float& ri) {
  static_assert(W == 4 || W == 16, "rows of a quad or of a 16-lane row");
  if constexpr (W == 4) {
    const float t = -ri;
    const float fn = t > 0.f ? t : 0.f;
    const float d = fn - fi;
    fi = (l == II) ? fn : fi;
    ri = fmaf_(a, group_bcast<II, W>(d), ri);
  } else {
    float fn, d;
    __asm__("v_max_f32_e64 %2, -%1, 0\n\t"
            "v_sub_f32_e32 %3, %2, %0\n\t"
            "v_cndmask_b32_e64 %0, %0, %2, %5\n\t"
            "s_nop 0\n\t"
            "v_fmac_f32_dpp %1, %3, %4 row_newbcast:%6 row_mask:0xf bank_mask:0xf"
            : "+v"(fi), "+v"(ri), "=&v"(fn), "=&v"(d)
            : "v"(a), "s"(lanes), "n"(II & 15));
  }
}

template <int II, int W>
__device__ __forceinline__ void pgs_sweep(const float (&Acol)[kMaxEfc], int l, unsigned long long lanes0, int nefc_max,
                                          float& fi, float& ri) {
  if constexpr (II < W) {
    if (II % 4 != 0 || II < nefc_max) {
      pgs_row<II, W>(Acol[II], l, lanes0 << II, fi, ri);
      pgs_sweep<II + 1, W>(Acol, l, lanes0, nefc_max, fi, ri);
    }
  }
}

// The sweep for worlds of up to 32 rows in paired-row form: lane l of a group holds two rows of its
// world, lo = l mod 16 and hi = 16 + l mod 16 (their scaled rows p and q, residuals and f), and both
// 16-lane rows of the group hold the same copy. Row II's change d then sits in lane II mod 16 of
// every 16-lane row, so one DPP row_newbcast inside each of the two fmas (r_lo += p_II d,
// r_hi += q_II d) broadcasts it: 5 VALU per row, where one row per lane needs a cross-row exchange
// (v_permlane16_swap, its register copy and wait states) on every row. Same operations in the same
// order as one row per lane, so the same values.
template <int II>
__device__ __forceinline__ void pgs_row_pair(float p, float q, unsigned long long lanes, float& fown, float& rlo,
                                             float& rhi) {
  float fn, d;
  if constexpr (II < 16) {
    __asm__("v_max_f32_e64 %3, -%1, 0\n\t"
            "v_sub_f32_e32 %4, %3, %0\n\t"
            "v_cndmask_b32_e64 %0, %0, %3, %7\n\t"
            "s_nop 0\n\t"
            "v_fmac_f32_dpp %1, %4, %5 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %2, %4, %6 row_newbcast:%8 row_mask:0xf bank_mask:0xf"
            : "+v"(fown), "+v"(rlo), "+v"(rhi), "=&v"(fn), "=&v"(d)
            : "v"(p), "v"(q), "s"(lanes), "n"(II & 15));
  } else {
    __asm__("v_max_f32_e64 %3, -%2, 0\n\t"
            "v_sub_f32_e32 %4, %3, %0\n\t"
            "v_cndmask_b32_e64 %0, %0, %3, %7\n\t"
            "s_nop 0\n\t"
            "v_fmac_f32_dpp %1, %4, %5 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %2, %4, %6 row_newbcast:%8 row_mask:0xf bank_mask:0xf"
            : "+v"(fown), "+v"(rlo), "+v"(rhi), "=&v"(fn), "=&v"(d)
            : "v"(p), "v"(q), "s"(lanes), "n"(II & 15));
  }
}

template <int II>
__device__ __forceinline__ void pgs_sweep_pair(const float (&P)[kMaxEfc], const float (&Q)[kMaxEfc],
                                               unsigned long long lanes0, int nefc_max, float& flo, float& fhi,
                                               float& rlo, float& rhi) {
  if constexpr (II < kMaxEfc) {
    if (II % 4 != 0 || II < nefc_max) {
      if constexpr (II < 16) pgs_row_pair<II>(P[II], Q[II], lanes0 << II, flo, rlo, rhi);
      else pgs_row_pair<II>(P[II], Q[II], lanes0 << (II - 16), fhi, rlo, rhi);
      pgs_sweep_pair<II + 1>(P, Q, lanes0, nefc_max, flo, fhi, rlo, rhi);
    }
  }
}

// Lane 0 of every 16-lane row: the row lanes of a sweep's first row (pgs_row, pgs_row_pair).
constexpr unsigned long long kPgsLanes0 = 0x0001000100010001ull;

// Sweeps between the fresh residuals of the PGS (a fresh residual r_i = c_i + sum_k a_ik f_k, k in
// order, bounds the rounding the row updates carry over long solves).
constexpr int kPgsRefresh = 8;

// Free joint of one M^-1 solve column (reference: src/aba_factor.cuh:139-155): D qdd = x_b -
// S_base.pA_1 with the factored D = L L' in LDS (forward, then backward substitution, each quotient
// by div_rn), then the pelvis acceleration a1 = S_base qdd (see sbase_dot / sbase_col).
__device__ __forceinline__ void base_solve(const WorldLds& s, const float (&xb)[6], const float (&p1)[6],
                                           float (&qdd)[6], float (&a1)[6]) {
  float rhs6[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) rhs6[k] = xb[k] - sbase_dot(k, s.u.fac.S[k], p1);
  const float* Lf = s.u.fac.Dfac;
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    float a = rhs6[i];
#pragma unroll
    for (int k = 0; k < i; ++k) a = fmaf_(-Lf[i * 6 + k], qdd[k], a);
    qdd[i] = div_rn(a, Lf[i * 6 + i], s.u.fac.Dinv[i]);
  }
#pragma unroll
  for (int i = 5; i >= 0; --i) {
    float a = qdd[i];
#pragma unroll
    for (int k = i + 1; k < 6; ++k) a = fmaf_(-Lf[k * 6 + i], qdd[k], a);
    qdd[i] = div_rn(a, Lf[i * 6 + i], s.u.fac.Dinv[i]);
  }
  float S3[3][3];
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int i = 0; i < 3; ++i) S3[k][i] = s.u.fac.S[3 + k][i];
#pragma unroll
  for (int i = 0; i < 6; ++i) a1[i] = sbase_col(i, S3, qdd);
}

// Ordering point between the phases of world_qacc, whose callers run it in workgroups of one wave
// (k_physics, k_rollout, k_probe: 64 threads). A wave's LDS accesses are performed in program
// order, so a wavefront-scope fence (the compiler keeps the accesses in order; no instruction) is
// all a hand-over through LDS between its lanes needs; __syncthreads() adds an lgkmcnt(0) drain of
// every outstanding LDS access at each phase boundary. The translation unit of k_rollout defines
// G1_PHASE_FENCE and takes the fence: config 3 10.50 -> 10.43 ms; k_physics keeps the barrier
// (with the default scheduler it was faster, 194.4 against 193.3 ms at config 4; with the ILP-first
// one both measure the same).
#ifdef G1_PHASE_FENCE
__device__ __forceinline__ void wave_sync() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }
#else
__device__ __forceinline__ void wave_sync() { __syncthreads(); }
#endif

// The chain layout's stores without a lane test (the factor, the force gather, the RNE staging): a
// chain outside its depth range writes the row of body c_off + depth, which its owner must store
// again later in the same sweep: in the leaf -> root sweeps above the torso depth (the legs past
// their leaf) at a smaller depth, in the root -> leaf RNE staging up to depth 7 (the right arm before
// its first body) at a larger one. Chain g: c_off, first and last depth as in world_qacc.
constexpr bool chain_stray_rows_rewritten() {
  const int off[4] = {0, 6, 12, 19}, lo[4] = {2, 2, 2, 5}, hi[4] = {7, 7, kMaxDepth, kMaxDepth};
  for (int g = 0; g < 4; ++g) {
    for (int cd = hi[g] + 1; cd <= kMaxDepth; ++cd)
      if (cd > body_depth[16] && !(body_depth[off[g] + cd] < cd)) return false;
    for (int r = 2; r < lo[g] && r <= 7; ++r)
      if (!(body_depth[off[g] + r] > r)) return false;
  }
  return true;
}
static_assert(chain_stray_rows_rewritten(), "rows stored outside a chain's range are stored again by their owners");

constexpr bool hinge_armature_uniform() {
  for (int d = 7; d < kNV; ++d)
    if (MF::dof_armature[d] != MF::dof_armature[6]) return false;
  return true;
}

// ================================================================ substep: qacc of one world
// Inputs: lane state, PD torque of the lane's hinge dof (jtau). Output: qacc of the lane's dofs
// (every lane: the 6 base dofs into bqacc[]; hinge lanes: jqacc). Returns this world's contact count.
// Must be called by all 64 lanes of the block in uniform control flow.
__device__ __forceinline__ int world_qacc(int lane, WorldLds& s, const LaneState& st, float jtau,
                                          const SolveParams& P, float (&bqacc)[6], float& jqacc) {
  // The lane index goes through an opaque asm on every call so the per-lane model constants are
  // re-read from the (cached) tables each substep instead of being hoisted out of the caller's
  // substep loop, where they would occupy ~150 registers for the whole kernel.
  int l = lane;
  __asm__ volatile("" : "+v"(l));
  const LaneModel L = lane_model(l);
  const bool base = (l == 1);
  // The lane's FK ancestor word (one byte per doubling round) and foot sphere (local position,
  // invweight0), read from its row with the lane model, so that their latency passes under the
  // hinge sincos instead of stalling the phase that uses them.
  const LaneRow R = lane_row(l);
  const unsigned anc = R.anc;
  const int sph = l < kNFoot ? l : 0;
  const V3 foot_lp{R.foot_lp[0], R.foot_lp[1], R.foot_lp[2]};
  const float foot_w0 = R.foot_w0;

  // ---------------- forward kinematics (reference: src/dynamics.cuh:47-88) by ancestor doubling
  // Each lane starts from its body's transform relative to its parent (hinge: translation
  // body_pos, rotation body_quat (x) the joint rotation; pelvis: the free-joint pose), and round r
  // composes it with the transform held by the 2^r-th ancestor, T <- T_anc o T, which leaves it
  // relative to the 2^(r+1)-th ancestor; after kFkRounds rounds every body is in the world frame.
  // The same per-body transforms as the reference's root -> leaf recursion, associated as a tree
  // (4 rounds instead of 10 levels); the CPU oracle composes in the same association. Hinge
  // anchors sit at the body origin (jnt_pos == 0, generator-checked), so the reference's anchor
  // shift pos = (pos + q*0) - q'*0 is the identity and is omitted.
  // The per-body transforms are formed in fp32, the compositions of every round but the last run in
  // fp64 and the frames are rounded to fp32 once before the last round (which only the arms' distal
  // links need; it and the inertial-frame offset run in fp32): the foot-ground contact is stiff in the foot
  // height, and fp64 compositions halve the fp32 error against MuJoCo's contact fixture (1.3e-5
  // against 2.9e-5 for fp32 doubling and 2.2e-5 for the reference's fp32 recursion). fp64 FMAs
  // issue like fp32 ones and take about twice their VALU time.
  V3 xp{0.f, 0.f, 0.f};
  Q4 xq{1.f, 0.f, 0.f, 0.f};
  V3 xip{0.f, 0.f, 0.f};
  {
    const float h = 0.5f * st.jq;
    float sn, cs;
    sincos_hinge_rn(h, sn, cs);
    const Q4 aa{cs, L.axis.x * sn, L.axis.y * sn, L.axis.z * sn};
    if (L.hinge) {
      xp = L.bpos;
      xq = qmul(L.bquat, aa);
    }
  }
  // the pelvis' orientation, on every lane (every lane carries the free joint's state)
  const Q4 qpel = qnorm(Q4{st.bq[3], st.bq[4], st.bq[5], st.bq[6]});
  if (base) {
    xp = {st.bq[0], st.bq[1], st.bq[2]};
    xq = qpel;
  }
  {
    V3d dp{xp.x, xp.y, xp.z};
    Q4d dq{xq.w, xq.x, xq.y, xq.z};
#pragma unroll
    for (int r = 0; r < kFkRounds - 1; ++r) {
      const int an = (anc >> (8 * r)) & 0xff;
      Q4d qa;
      V3d pa;
      if (r == 0) {
        // the parents' transforms are still the fp32 ones, exactly widened: move the floats (7 lane
        // exchanges instead of 14) and widen after the move
        qa = {gshfl(xq.w, an), gshfl(xq.x, an), gshfl(xq.y, an), gshfl(xq.z, an)};
        pa = {gshfl(xp.x, an), gshfl(xp.y, an), gshfl(xp.z, an)};
      } else {
        qa = {gshfld(dq.w, an), gshfld(dq.x, an), gshfld(dq.y, an), gshfld(dq.z, an)};
        pa = {gshfld(dp.x, an), gshfld(dp.y, an), gshfld(dp.z, an)};
      }
      // Every lane composes, also where the 2^r-th ancestor would lie beyond the world: there `an`
      // is 0, the world body's lane, whose transform is the identity (zero translation, quaternion
      // (1, 0, 0, 0)) and stays exactly that under its own compositions. Composing with it returns
      // the transform unchanged except for the sign of an exact zero, and the CPU restatement
      // composes the same way: no branch and no selects around the composition.
      dp = vaddd(pa, qrotd(qa, dp));
      dq = qmuld(qa, dq);
    }
    // The last round in fp32, on the frames rounded once: only the arms' distal bodies (depth >=
    // 2^(kFkRounds-1) + 1) have an ancestor left, and every other lane composes with the world's
    // identity, which is exact, so its frame (the feet's among them) is the fp64 one rounded once.
    // The inertial-frame offset then follows in fp32 from the final frame.
    static_assert(body_depth[foot_body[0]] <= (1 << (kFkRounds - 1)) &&
                  body_depth[foot_body[kNFoot - 1]] <= (1 << (kFkRounds - 1)), "the feet are final before the fp32 round");
    xp = {(float)dp.x, (float)dp.y, (float)dp.z};
    xq = {(float)dq.w, (float)dq.x, (float)dq.y, (float)dq.z};
    {
      const int an = (anc >> (8 * (kFkRounds - 1))) & 0xff;
      const Q4 qa{gshfl(xq.w, an), gshfl(xq.x, an), gshfl(xq.y, an), gshfl(xq.z, an)};
      const V3 pa{gshfl(xp.x, an), gshfl(xp.y, an), gshfl(xp.z, an)};
      xp = vadd(pa, qrot(qa, xp));
      xq = qmul(qa, xq);
    }
    xip = vadd(xp, qrot(xq, L.ipos));
  }
  // pelvis origin: every lane carries the free joint's state (integrate_lane), and the pelvis' frame
  // is its position as it stands (no ancestor to compose with)
  const V3 p{st.bq[0], st.bq[1], st.bq[2]};

  // ---------------- contact detection: lane s = foot sphere s (reference: src/contact.cuh:31-46)
  int ncon = 0;
  if (P.contact) {
    // spheres 0..3 on the left foot, 4..7 on the right
    static_assert(foot_body[0] == foot_body[kNFoot / 2 - 1] && foot_body[kNFoot / 2] == foot_body[kNFoot - 1],
                  "foot spheres in two halves");
    const int fb = sph < kNFoot / 2 ? foot_body[0] : foot_body[kNFoot - 1];
    // the foot bodies' lanes lie in the sphere lanes' 16-lane row: their frames by DPP row
    // broadcasts and a select instead of lane exchanges through LDS
    static_assert(foot_body[0] < 16 && foot_body[kNFoot - 1] < 16 && kNFoot <= 16, "feet in row 0");
    constexpr int kL = foot_body[0], kR = foot_body[kNFoot - 1];
    const bool left = sph < kNFoot / 2;
    // (both broadcasts on every lane before the select: a DPP move inside a lane-divergent branch
    // would read a source lane that the branch has switched off)
    auto foot = [&](float v) {
      float a = group_bcast<kL, 16>(v), b = group_bcast<kR, 16>(v);
      __asm__ volatile("" : "+v"(a), "+v"(b));
      return left ? a : b;
    };
    Q4 fq{foot(xq.w), foot(xq.x), foot(xq.y), foot(xq.z)};
    V3 fp{foot(xp.x), foot(xp.y), foot(xp.z)};
    V3 c = vadd(fp, qrot(fq, foot_lp));
    const float pen = c.z - MF::foot_radius;
    const bool hit = (l < kNFoot) && (pen < 0.f);
    const unsigned mask = group_ballot8(hit);
    ncon = __popc(mask);
    if (hit) {
      const int idx = __popc(mask & ((1u << l) - 1u));
      s.con[idx][0] = c.x; s.con[idx][1] = c.y; s.con[idx][2] = pen * 0.5f; s.con[idx][3] = pen;
      s.con_w0[idx] = foot_w0;
      s.con_leg[idx] = (fb == foot_body[kNFoot - 1]) ? 1 : 0;
    }
  }
  // (detected right after FK: the contact count decides below who computes the smooth solve's
  // base and root -> leaf parts; the LDS writes are read after the later barriers)
  const int ncon_max = groups_max(ncon);

  // ---------------- motion axes (reference: src/aba_bias.cuh:25-43)
  V3 sw{0.f, 0.f, 0.f}, sv{0.f, 0.f, 0.f};   // hinge axis (angular; linear)
  // the pelvis rotation on every lane (the free joint's right-hand side and base solve use it)
  const M3 R1 = quat2mat(qpel);
  if (L.hinge) {
    sw = qrot(xq, L.axis);
    sv = cross(vsub(xp, p), sw);
    const int d = L.b + 4;
    s.u.fac.S[d][0] = sw.x; s.u.fac.S[d][1] = sw.y; s.u.fac.S[d][2] = sw.z;
    s.u.fac.S[d][3] = sv.x; s.u.fac.S[d][4] = sv.y; s.u.fac.S[d][5] = sv.z;
    s.u.fac.S[d][6] = L.bdt;   // the row's padding carries the factor's dt kd (column 7: x_b)
    s.qvel[d] = st.jqd;
  }
  if (base) {
    // only the rotations' angular parts (R1 columns) are stored: every use of the free joint's
    // subspace takes its structure from sbase_dot / sbase_col
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      s.u.fac.S[3 + k][0] = R1.m[k]; s.u.fac.S[3 + k][1] = R1.m[3 + k]; s.u.fac.S[3 + k][2] = R1.m[6 + k];
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) s.qvel[k] = st.bqd[k];
  }

  // ---------------- body inertia about the pelvis origin (reference: src/aba_bias.cuh:45-55)
  M3 Iw;
  V3 cc{0.f, 0.f, 0.f};
  {
    M3 Ri = quat2mat(qmul(xq, L.iquat));
    const float d[3] = {L.inert.x, L.inert.y, L.inert.z};
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j)
        Iw.m[3 * i + j] = fmaf_(Ri.m[3 * i + 2] * d[2], Ri.m[3 * j + 2],
                                fmaf_(Ri.m[3 * i + 1] * d[1], Ri.m[3 * j + 1], Ri.m[3 * i + 0] * d[0] * Ri.m[3 * j + 0]));
    cc = vsub(xip, p);
  }
  const float m = L.body ? L.mass : 0.f;

  // ---------------- RNE velocities / accelerations, qacc = 0 (reference: src/aba_bias.cuh:57-102)
  V3 vw{0.f, 0.f, 0.f}, vv{0.f, 0.f, 0.f}, aw{0.f, 0.f, 0.f}, av{0.f, 0.f, 0.f};
  if (l == 0) av = {-MF::gravity[0], -MF::gravity[1], -MF::gravity[2]};
  if (base) {
    // free joint: translations accumulate normally; the three rotational cdof_dot use the
    // post-translation partial velocity (reference: src/aba_bias.cuh:68-85). With the subspace's
    // structural zeros skipped (see sbase_dot): the translations leave w = 0, v = (qd0, qd1, qd2)
    // and cdof_dot = 0; rotation k has cdof_dot = (0, v x R1 col k), and w sums R1 col k qd(3+k)
    const V3 vr{st.bqd[0], st.bqd[1], st.bqd[2]};
    V3 w{R1.m[0] * st.bqd[3], R1.m[3] * st.bqd[3], R1.m[6] * st.bqd[3]};
    V3 a_v{-MF::gravity[0], -MF::gravity[1], -MF::gravity[2]};
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const V3 Rk{R1.m[k], R1.m[3 + k], R1.m[6 + k]};
      const float qd = st.bqd[3 + k];
      if (k > 0) w = {fmaf_(Rk.x, qd, w.x), fmaf_(Rk.y, qd, w.y), fmaf_(Rk.z, qd, w.z)};
      const V3 sdv = cross(vr, Rk);
      a_v = {fmaf_(sdv.x, qd, a_v.x), fmaf_(sdv.y, qd, a_v.y), fmaf_(sdv.z, qd, a_v.z)};
    }
    vw = w; vv = vr;
    aw = {0.f, 0.f, 0.f}; av = a_v;
  }
  // Hinge bodies, chain-parallel: the hinges form four chains (left leg 2..7, right leg 8..13,
  // waist 14..16 continued by the left arm 17..23, right arm 24..30 off the torso 16), walked
  // root -> leaf in lock-step over tree depth. Chain g runs on lanes 8g..8g+5 and lane 8g+c holds
  // spatial component c (w0 w1 w2 v0 v1 v2) of the current body's velocity and acceleration; the
  // cross products take the parent's other components from the chain's lanes. Each component is
  // the lane-per-body formula term for term: v = vp + S qd, a = ap + (vp x S) qd with
  // (vp x S)_w = w_p x s_w, (vp x S)_v = w_p x s_v + v_p x s_w. The results go to LDS (the
  // solve-output region is idle until the factor) and each body lane reads its own back.
  const int grp = l >> 3, crow = l & 7, rowc = crow < 6 ? crow : 5;
  const int c_off = grp == 0 ? 0 : (grp == 1 ? 6 : (grp == 2 ? 12 : 19));
  const int c_lo = grp == 3 ? 5 : 2, c_hi = grp >= 2 ? kMaxDepth : 7;
  // Body of chain g at depth cd. Outside the chain's depth range this is another in-range body
  // (cd + c_off lies in 1..30 for every cd in 1..11) whose data is read, and stored only where its
  // owner stores it again later in the sweep (chain_stray_rows_rewritten): keeping the index linear
  // in cd lets every per-level LDS address be a loop-invariant register plus an immediate offset.
  auto chain_body = [&](int cd) { return cd + c_off; };
  constexpr int kTorsoDepth = body_depth[16];   // the arms' parent, the waist chain's last body
  static_assert(kMaxDepth + 19 < kNBody, "chain bodies in range");
  static_assert(body_parent[2] == 1 && body_parent[8] == 1 && body_parent[14] == 1 && body_parent[24] == 16 &&
                body_depth[24] == 5 && body_depth[2] == 2, "chain roots");
  // body velocity and acceleration about the pelvis origin, interleaved per body (w, v of the
  // velocity, two floats of padding where chain lanes 6 and 7 store, the acceleration likewise, four
  // more): every level's slot sits at an immediate offset from the lane's base, and the body stride
  // of 20 words puts the four chains' rows of a level on different LDS banks
  constexpr int kVA = 20;
  float* const V6 = &s.Mm[0][0];
  float* const A6 = V6 + kVA / 2;
  static_assert(kCols * kMmStride >= kNBody * kVA && kVA / 2 >= 8, "RNE staging fits the solve-output region");
  if (base) {
    V6[kVA + 0] = vw.x; V6[kVA + 1] = vw.y; V6[kVA + 2] = vw.z; V6[kVA + 3] = vv.x; V6[kVA + 4] = vv.y; V6[kVA + 5] = vv.z;
    A6[kVA + 0] = aw.x; A6[kVA + 1] = aw.y; A6[kVA + 2] = aw.z; A6[kVA + 3] = av.x; A6[kVA + 4] = av.y; A6[kVA + 5] = av.z;
  }
  wave_sync();   // pelvis velocity / acceleration and every motion axis and hinge qvel in LDS
  {
    const int k = rowc < 3 ? rowc : rowc - 3, k1 = k == 2 ? 0 : k + 1, k2 = k == 0 ? 2 : k - 1;
    const bool isv = rowc >= 3;
    const int so = isv ? 3 : 0;
    // per-lane base pointers: depth r's operands sit at a constant offset from them
    const float* const Sl = &s.u.fac.S[c_off + 4][0];
    const float* const pS0 = Sl + rowc;
    const float* const pS1 = Sl + so + k1;
    const float* const pS2 = Sl + so + k2;
    const float* const pS3 = Sl + k1;
    const float* const pS4 = Sl + k2;
    const float* const pq = &s.qvel[c_off + 4];
    float* const pV = V6 + kVA * c_off + crow;
    float* const pA = A6 + kVA * c_off + crow;
    // The velocities first: v = vp + S qd is a sum per component, so lane rowc needs nothing from
    // the other lanes of its chain (the right arm's first body takes the torso's component from
    // chain 2's lanes by row_shr:8); every level's operands are read before the sweep.
    float Sr[kMaxDepth + 1], qd[kMaxDepth + 1];
#pragma unroll
    for (int r = 2; r <= kMaxDepth; ++r) { Sr[r] = pS0[kRow * r]; qd[r] = pq[r]; }
    float pc = V6[kVA + rowc];   // component rowc of the current body's v (the pelvis' first)
#pragma unroll
    for (int r = 2; r <= kMaxDepth; ++r) {
      const bool act = r >= c_lo && r <= c_hi;
      float P = pc;
      if (r == kTorsoDepth + 1) {
        const float t = from_prev_chain(pc);   // chain 2 -> 3: the torso's component
        P = grp == 3 ? t : pc;
      }
      // a chain's values outside its depth range are never read (its first body takes the parent
      // from the pelvis or the torso), so no select keeps them
      pc = fmaf_(Sr[r], qd[r], P);
      // Stores: lanes 6 and 7 into the padding. Up to depth 7 every lane stores: the only inactive
      // chain there, the right arm before its first body (depths 2..4), writes rows 21..23, which
      // chain 2 stores again at depths 9..11. Beyond depth 7 the legs are past their last body and
      // would overwrite rows that chains 1 and 2 stored at depths 2..5, so `act` guards.
      if (r <= 7 || act) pV[kVA * r] = pc;
    }
    // Then the accelerations a = ap + (vp x S) qd: the cross products take the parent's other
    // components from its velocity row as just stored (four reads at per-lane columns; at depth 2
    // the pelvis' row, for the right arm's first body the torso's, chain 2's depth-4 row). Those
    // reads do not wait on the acceleration chain, so only one fma per level is serial; each
    // level's operands are read two levels ahead.
    auto ldc = [&](int r, float (&o)[8]) {
      const float* const prow = r == 2 ? V6 + kVA
                                       : (r == kTorsoDepth + 1 && grp == 3 ? V6 + kVA * 16 : V6 + kVA * (c_off + r - 1));
      o[0] = prow[k1]; o[1] = prow[k2];           // w_p[k+1], w_p[k+2]
      o[2] = prow[3 + k1]; o[3] = prow[3 + k2];   // v_p[k+1], v_p[k+2]
      o[4] = pS1[kRow * r]; o[5] = pS2[kRow * r]; o[6] = pS3[kRow * r]; o[7] = pS4[kRow * r];
    };
    float cur[8], nxt[8];
    ldc(2, cur);
    ldc(3, nxt);
    float pac = A6[kVA + rowc];   // component rowc of the current body's a (the pelvis' first)
#pragma unroll
    for (int r = 2; r <= kMaxDepth; ++r) {
      const bool act = r >= c_lo && r <= c_hi;
      float nn[8];
      if (r + 2 <= kMaxDepth) ldc(r + 2, nn);
      const float X1 = cur[0], X2 = cur[1], Y1 = cur[2], Y2 = cur[3];
      const float Sw1 = cur[4], Sw2 = cur[5], Sv1 = cur[6], Sv2 = cur[7];
      const float t1 = fmaf_(-X2, Sw1, X1 * Sw2);   // (w_p x s_w)_k, or (w_p x s_v)_k
      const float t2 = fmaf_(-Y2, Sv1, Y1 * Sv2);   // (v_p x s_w)_k
      const float sd = isv ? t1 + t2 : t1;
      float PA = pac;
      if (r == kTorsoDepth + 1) {
        const float t = from_prev_chain(pac);   // chain 2 -> 3: the torso's component
        PA = grp == 3 ? t : pac;
      }
      pac = fmaf_(sd, qd[r], PA);
      if (r <= 7 || act) pA[kVA * r] = pac;
#pragma unroll
      for (int e = 0; e < 8; ++e) { cur[e] = nxt[e]; nxt[e] = nn[e]; }
    }
  }
  wave_sync();
  if (L.hinge) {
    const float* v6 = V6 + kVA * L.b;
    const float* a6 = A6 + kVA * L.b;
    vw = {v6[0], v6[1], v6[2]}; vv = {v6[3], v6[4], v6[5]};
    aw = {a6[0], a6[1], a6[2]}; av = {a6[3], a6[4], a6[5]};
  }

  // ---------------- body forces f = I a + v x* (I v) (reference: src/aba_bias.cuh:103-111,
  // inertia application src/dynamics.cuh:126-139)
  auto apply_I = [&](V3 xw, V3 xv, V3& fw, V3& fv) {
    V3 Asw{fmaf_(Iw.m[2], xw.z, fmaf_(Iw.m[1], xw.y, Iw.m[0] * xw.x)),
           fmaf_(Iw.m[5], xw.z, fmaf_(Iw.m[4], xw.y, Iw.m[3] * xw.x)),
           fmaf_(Iw.m[8], xw.z, fmaf_(Iw.m[7], xw.y, Iw.m[6] * xw.x))};
    const float c2 = dot3(cc, cc), csw = dot3(cc, xw);
    Asw = {fmaf_(m, fmaf_(-csw, cc.x, c2 * xw.x), Asw.x), fmaf_(m, fmaf_(-csw, cc.y, c2 * xw.y), Asw.y),
           fmaf_(m, fmaf_(-csw, cc.z, c2 * xw.z), Asw.z)};
    V3 mc = cross(cc, xv);
    fw = {fmaf_(m, mc.x, Asw.x), fmaf_(m, mc.y, Asw.y), fmaf_(m, mc.z, Asw.z)};
    V3 cs = cross(cc, xw);
    fv = {fmaf_(m, xv.x, -m * cs.x), fmaf_(m, xv.y, -m * cs.y), fmaf_(m, xv.z, -m * cs.z)};
  };
  V3 Fw{0.f, 0.f, 0.f}, Fv{0.f, 0.f, 0.f};
  if (L.body) {
    V3 Iaw, Iav, Ivw, Ivv;
    apply_I(aw, av, Iaw, Iav);
    apply_I(vw, vv, Ivw, Ivv);
    V3 a = cross(vw, Ivw), b = cross(vv, Ivv);
    V3 cw{a.x + b.x, a.y + b.y, a.z + b.z};
    V3 cv = cross(vw, Ivv);
    Fw = {Iaw.x + cw.x, Iaw.y + cw.y, Iaw.z + cw.z};
    Fv = {Iav.x + cv.x, Iav.y + cv.y, Iav.z + cv.z};
  }
  // ---------------- body spatial inertia about the pelvis origin (reference:
  // src/aba_factor.cuh:51-76), staged in LDS for the chain-parallel factor as full rows: entry
  // (i, j) holds the packed upper-triangle value (min(i, j), max(i, j)), the reference's 21 numbers,
  // so that a factor lane reads its row with three 8-byte reads instead of six scattered ones.
  // The bodies' own forces go to the hinge-factor column rows (U), which the factor overwrites only
  // for the hinge bodies 2..30: the pelvis' subtree force (row 1) is read after the factor.
  static_assert(sizeof(float) * kNBody * kRow >= sizeof(float) * kNBody * 6, "force staging fits U");
  float* const Fo = &s.u.fac.U[0][0];     // [kNBody][6] each body's own RNE force (w, v)
  if (L.body) {
    Fo[6 * L.b + 0] = Fw.x; Fo[6 * L.b + 1] = Fw.y; Fo[6 * L.b + 2] = Fw.z;
    Fo[6 * L.b + 3] = Fv.x; Fo[6 * L.b + 4] = Fv.y; Fo[6 * L.b + 5] = Fv.z;
  }
  if (L.body) {
    const float c2 = dot3(cc, cc);
    float A[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) A[i] = Iw.m[i];
    A[0] = fmaf_(m, fmaf_(-cc.x, cc.x, c2), A[0]); A[1] = fmaf_(m, -cc.x * cc.y, A[1]); A[2] = fmaf_(m, -cc.x * cc.z, A[2]);
    A[3] = fmaf_(m, -cc.y * cc.x, A[3]); A[4] = fmaf_(m, fmaf_(-cc.y, cc.y, c2), A[4]); A[5] = fmaf_(m, -cc.y * cc.z, A[5]);
    A[6] = fmaf_(m, -cc.z * cc.x, A[6]); A[7] = fmaf_(m, -cc.z * cc.y, A[7]); A[8] = fmaf_(m, fmaf_(-cc.z, cc.z, c2), A[8]);
    const float Bx[9] = {0.f, -cc.z, cc.y, cc.z, 0.f, -cc.x, -cc.y, cc.x, 0.f};
    float M6[36];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        M6[6 * i + j] = A[3 * i + j];
        M6[6 * i + (j + 3)] = m * Bx[3 * i + j];
        M6[6 * (i + 3) + j] = -m * Bx[3 * i + j];
        M6[6 * (i + 3) + (j + 3)] = (i == j) ? m : 0.f;
      }
#pragma unroll
    for (int i = 0; i < 6; ++i)
#pragma unroll
      for (int j = 0; j < 6; ++j) s.I6r[L.b][i][j] = M6[(i <= j ? i : j) * 6 + (i <= j ? j : i)];
  }
  wave_sync();   // S, I6 and the own forces of every body in LDS

  // ---------------- RNE force gather (reference: src/aba_bias.cuh:112-120), chain-parallel, and
  // the hinge right-hand sides x_b = tau_b - S_b.F_b of the smooth solve. Lane (chain g, row r)
  // carries component r of the subtree force F_b = F_own_b + the children's F in descending child
  // order (torso: + F_24 then + F_17), walked leaf -> root in lock-step over depth in the factor's
  // layout below, and overwrites F_own_b in place; the pelvis' F_1 = F_own_1 + F_14 + F_8 + F_2
  // closes the sweep. The chain is one addition per level with no exchange inside the chain, and
  // each hinge lane then takes its own body's F from LDS for S_b.F_b (the lane-per-body form's
  // order), so the factor's sweep only reads x_b.
  {
    float* const pF = Fo + 6 * c_off + rowc;
    // every level's own force read before the sweep (each level reads its own slot once, before
    // it stores it): the reads go out together instead of one LDS round trip per level, which the
    // stores' branches kept the scheduler from overlapping
    float Fl[kMaxDepth + 1];
#pragma unroll
    for (int cd = kMaxDepth; cd >= 2; --cd) Fl[cd] = pF[6 * cd];
    float Fc = 0.f;   // component rowc of the last body's subtree force
#pragma unroll
    for (int cd = kMaxDepth; cd >= 2; --cd) {
      const bool act = cd >= c_lo && cd <= c_hi;
      float F = Fl[cd];
      if (cd == kTorsoDepth) {
        // the right arm (chain 3) ends at depth 5; its force joins the torso (chain 2) first
        const float g24 = from_next_chain(Fc);
        F = grp == 2 ? F + g24 : F;
      }
      F = cd == c_hi ? F : F + Fc;
      // lanes 6 and 7 of a chain repeat row 5 (rowc) and store the same value to the same slot.
      // From depth 5 up every lane stores: the legs past their last body (depths 8..11) write
      // rows 8..11 and 14..17, which chains 1 and 2 store again at depths 2..5 (every own force was
      // read before the sweep); below, the right arm past its root would overwrite rows 21..23.
      if (cd > kTorsoDepth || act) pF[6 * cd] = F;
      Fc = F;
    }
    // pelvis, component r on lane r of chain 0 (chain 2's and chain 1's roots reach chain 0's
    // lanes by v_permlane16_swap and row_shl:8)
    const float F1 = ((Fo[6 + rowc] + from_upper_row(Fc)) + from_next_chain(Fc)) + Fc;
    if (l < 6) Fo[6 + l] = F1;
  }
  wave_sync();   // every subtree force in LDS
  if (L.hinge) {
    const float* const Fb = Fo + 6 * L.b;
    const float* const Sb = s.u.fac.S[L.b + 4];   // (w, v) of the hinge axis, as stored above
    float bias = Sb[0] * Fb[0];
#pragma unroll
    for (int j = 1; j < 6; ++j) bias = fmaf_(Sb[j], Fb[j], bias);
    s.u.fac.S[L.b + 4][7] = -bias + jtau;   // x_b, beside the axis for the factor, which stores u_b = x_b - S_b.pA_b
  }
  wave_sync();

  // ---------------- damped articulated-inertia factor, chain-parallel (reference:
  // src/aba_factor.cuh:77-88), fused with the leaf -> root sweep of the smooth solve
  // y = (M + dtB)^-1 (tau - bias) (reference: src/aba_factor.cuh:128-136).
  // The hinge bodies form four chains processed leaf -> root in lock-step over tree depth cd:
  // left leg 7..2, right leg 13..8, left arm 23..17 then waist 16..14, right arm 30..24.
  // Chain g runs on lanes 8g..8g+5 of the group and lane 8g+r holds row r of the current body's
  // articulated inertia; U = I^A S is exchanged within the chain, D, the bias u and the
  // articulated bias force pA are computed redundantly by the six lanes. Every entry sees the
  // reference's operations in the reference's order: I^A_b = I6_b + the children's downdates in
  // descending child order (torso: + D_24 then + D_17), U_i = sum_j I^A_ij S_j, D = S.U + arm
  // (+ dt kd), downdate I^A_ij - U_i U_j / D; the products U_i U_j commute, so row r of the
  // symmetric downdate equals the packed entries bit for bit.
  float Dlr[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};   // row `crow` of the last body's downdate
  float cs[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};    // last body's pA + U u / D (all six components)
  // the next level's body inputs (motion axis, I6 row, right-hand side x_b, dt kd; the last two in
  // the axis row's padding), loaded while the current level computes
  float Sn[6], In[6], xn, kn;
  // every hinge has the same armature (the model's 0.01): a constant, not a per-body gather
  constexpr float kArm = MF::dof_armature[6];
  static_assert(hinge_armature_uniform(), "one armature for every hinge dof");
  // per-lane base pointers: depth cd's operands and results sit at constant offsets from them
  const float* const pSc = &s.u.fac.S[c_off + 4][0];
  const float* const pIc = &s.I6r[c_off][rowc][0];
  float* const pUc = &s.u.fac.U[c_off][crow];
  // two levels in flight: level cd computes from (Sn, In, xn, kn) while the next level's inputs
  // (Sm, Im, xm, km) arrive and the one after it is requested
  float Sm[6], Im[6], xm, km;
  static_assert(kRow == 8, "axis row: six components, dt kd, x_b");
  auto prefetch = [&](int cd) {
#pragma unroll
    for (int j = 0; j < 6; ++j) { Sn[j] = Sm[j]; In[j] = Im[j]; }
    xn = xm;
    kn = km;
#pragma unroll
    for (int j = 0; j < 6; ++j) { Sm[j] = pSc[kRow * cd + j]; Im[j] = pIc[36 * cd + j]; }
    km = pSc[kRow * cd + 6];
    xm = pSc[kRow * cd + 7];
  };
  // one level of the chains; `junction` adds the right arm's downdate and bias force (gD, gc)
  // to the torso before its own child's
  auto level = [&](int cd, bool junction, const float* gD, const float* gc) {
    const bool act = cd >= c_lo && cd <= c_hi;
    const bool leaf = cd == c_hi;
    float Sd[6], IAr[6], pA[6];
    const float xb_ = xn, arm = kArm, bdt = kn;
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      Sd[j] = Sn[j];
      // the bias force accumulates the children's terms from the first one (no 0 + x: a sum that
      // starts at the first term differs from 0 + ... only in the sign of an exact zero)
      float v = In[j];
      if (junction) v = v + gD[j];
      IAr[j] = leaf ? v : v + Dlr[j];
      pA[j] = leaf ? 0.f : (junction ? gc[j] + cs[j] : cs[j]);
    }
    // the inputs of two levels down, as soon as this level's are taken (depths 1 and 0 load
    // bodies that are never used)
    prefetch(cd - 2);
    float ur = 0.f;
#pragma unroll
    for (int j = 0; j < 6; ++j) ur = fmaf_(IAr[j], Sd[j], ur);
    const float Ub[6] = {chain_bcast<0>(ur), chain_bcast<1>(ur), chain_bcast<2>(ur),
                         chain_bcast<3>(ur), chain_bcast<4>(ur), chain_bcast<5>(ur)};
    float D = dot6(Sd, Ub) + arm;
    if (P.damped) D += bdt;
    const float invD = rcp_rn(D);
    const float u = xb_ - dot6(Sd, pA);
    const float ud = u * invD;
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const float dl = fmaf_(-(ur * Ub[j]), invD, IAr[j]);   // ur == Ub[crow] on rows 0..5
      const float c = fmaf_(Ub[j], ud, pA[j]);
      // Outside a chain's depth range its values are dead: before its leaf the leaf level starts
      // afresh, after its root nothing reads them (the right arm's last body is read at the
      // torso level before that level overwrites it); only the LDS stores below need `act`.
      Dlr[j] = dl;
      cs[j] = c;
    }
    // one store per level for the whole row: lanes 0..5 their column entry, lanes 6 and 7 (which
    // compute invD and u as the others do) the reciprocal pivot and the bias. From depth 5 up every
    // lane stores (the legs' rows beyond their leaf are stored again by chains 1 and 2 at depths
    // 2..5, and nothing reads U during the sweep); below, the right arm past its root would
    // overwrite rows 21..23.
    if (cd > kTorsoDepth || act) pUc[kRow * cd] = crow < 6 ? ur : (crow == kInvD ? invD : u);
  };
  // Issue priority (s_setprio): two waves share a SIMD, and the phases that are dependency chains
  // over the tree or the PGS rows (this factor: 1; the contact pipeline from PASS 1 through PGS: 3)
  // go ahead of the other wave's wider phases. Same-box A/B, ms per rollout: config 3 12.69 ->
  // 12.54, config 4 232.5 -> 230.1 (priority raised for FK or RNE as well was slower, for PGS
  // alone 12.64).
  __builtin_amdgcn_s_setprio(1);
  prefetch(kMaxDepth);
  prefetch(kMaxDepth - 1);
  const float none[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cd = kMaxDepth; cd > kTorsoDepth; --cd) level(cd, false, none, none);
  {
    // the right arm (chain 3, lanes 24..) ends at depth 5; its downdate and bias force join the
    // torso (chain 2) at depth 4
    static_assert(body_parent[24] == 16 && body_parent[17] == 16 && body_depth[24] == kTorsoDepth + 1, "torso");
    float gD[6], gc[6];   // chain 3's rows on chain 2's lanes (row_shl:8)
#pragma unroll
    for (int j = 0; j < 6; ++j) { gD[j] = from_next_chain(Dlr[j]); gc[j] = from_next_chain(cs[j]); }
    level(kTorsoDepth, grp == 2, gD, gc);
  }
#pragma unroll
  for (int cd = kTorsoDepth - 1; cd >= 2; --cd) level(cd, false, none, none);
  // pelvis: I^A_1 = I6_1 + D_14 + D_8 + D_2 and pA_1 = cs_14 + cs_8 + cs_2 (descending children),
  // row r on lane r of chain 0, which all hold pA_1
  float pAs[6], I1[6];
  float xb[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  {
    // the free joint's right-hand side -S_base.F_1 on every lane (F_1 from the force gather)
    {
      const V3 Fw{Fo[6], Fo[7], Fo[8]}, Fv{Fo[9], Fo[10], Fo[11]};
      // x_base = 0 - S_base.F_1 (see sbase_dot): translation k takes Fv_k, rotation k R1 col k . Fw
      xb[0] = -Fv.x; xb[1] = -Fv.y; xb[2] = -Fv.z;
#pragma unroll
      for (int k = 0; k < 3; ++k) xb[3 + k] = -fmaf_(R1.m[6 + k], Fw.z, fmaf_(R1.m[3 + k], Fw.y, R1.m[k] * Fw.x));
    }
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const float d14 = from_upper_row(Dlr[j]), d8 = from_next_chain(Dlr[j]);
      const float c14 = from_upper_row(cs[j]), c8 = from_next_chain(cs[j]);
      I1[j] = ((s.I6r[1][rowc][j] + d14) + d8) + Dlr[j];
      pAs[j] = (c14 + c8) + cs[j];
    }
  }
  __builtin_amdgcn_s_setprio(0);
  // ---------------- free-joint 6x6 block (reference: src/aba_factor.cuh:90-108): lane c < 6
  // builds column c of U6 = I^A S_base and of D = S_base' U6; every lane then factors D and solves
  // the base of the smooth system.
  // I^A rows from chain 0's lanes (lane r holds row r; I^A is symmetric bit for bit, the downdate
  // products commuting, so row r is also column r): lanes c < 3 take row 3 + c, their translation
  // column; lanes c >= 3 rows 0..2, the angular columns. Lane exchanges instead of a staging
  // round trip through LDS.
  float Ir[3][6];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int src = l < 3 ? (q == 0 ? 3 + l : 0) : q;
#pragma unroll
    for (int j = 0; j < 6; ++j) Ir[q][j] = gshfl(I1[j], src);
  }
  if (l < 6) {
    // column l of U6 = I^A S_base: translation l < 3 picks column 3 + l of I^A, rotation l >= 3
    // is I^A's angular columns times R1 col (l - 3) (structural zeros skipped, see sbase_dot). The
    // lane's rotation column is read at a lane-dependent LDS address rather than selected among
    // registers, which the compiler turned into divergent branches (an exec-mask diamond per select).
    float S3[3][3];   // S3[k][i] = S_base rotation k, component i = R1 column k
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
      for (int i = 0; i < 3; ++i) S3[k][i] = R1.m[3 * i + k];
    const int rl = l < 3 ? 0 : l - 3;   // the lane's rotation (translation lanes: row 0, unused)
    float Sc[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) Sc[i] = s.u.fac.S[3 + rl][i];
    float U6c[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const float rot = fmaf_(Ir[2][i], Sc[2], fmaf_(Ir[1][i], Sc[1], Ir[0][i] * Sc[0]));
      U6c[i] = l < 3 ? Ir[0][i] : rot;
    }
    // D = S_base' U6 (+ armature and dt*damping, both 0 on the free joint)
#pragma unroll
    for (int k = 0; k < 6; ++k) s.u.fac.Dm[k * 6 + l] = sbase_dot(k, S3[k < 3 ? 0 : k - 3], U6c);
  }
  // pA_1 from lane 1 (chain 0's lanes hold it) to every lane for the smooth base solve (waves
  // without contacts), while D is built and read
  float pA1[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (ncon_max == 0) {
#pragma unroll
    for (int k = 0; k < 6; ++k) pA1[k] = gshfl(pAs[k], 1);
  }
  wave_sync();
  // Every lane factors D and, without contacts, solves the base of the smooth system: the same
  // operations on the same values (D's lower triangle read whole, the same addresses on every lane;
  // S_base's rotation rows are R1's columns, on every lane), so that the base acceleration and
  // qacc are local to every lane for the root -> leaf sweep and the integration: no exec-mask region
  // and no lane exchange after the serial chain.
  float a6[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float qb[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};   // the smooth solve's base qacc (no contacts)
  {
    float Dm[36], Dinv[6];
#pragma unroll
    for (int i = 0; i < 6; ++i)
#pragma unroll
      for (int j = 0; j <= i; ++j) Dm[i * 6 + j] = s.u.fac.Dm[i * 6 + j];
#pragma unroll
    for (int i = 0; i < 6; ++i)
#pragma unroll
      for (int j = 0; j <= i; ++j) {
        float a = Dm[i * 6 + j];
#pragma unroll
        for (int k = 0; k < j; ++k) a = fmaf_(-Dm[i * 6 + k], Dm[j * 6 + k], a);
        if (i == j) {
          Dm[i * 6 + i] = sqrt_rn_pos(a);
          Dinv[i] = rcp_rn(Dm[i * 6 + i]);
        } else {
          Dm[i * 6 + j] = div_rn(a, Dm[j * 6 + j], Dinv[j]);
        }
      }
    // With contacts the smooth solve's base and root -> leaf parts run as column 0 of the contact
    // solves below (lane 0, the same operations in the same order), which read the factor from LDS
    // (the lower triangle); without, here and in the level-synchronous sweep.
    if (ncon_max > 0) {
      if (base) {
#pragma unroll
        for (int i = 0; i < 6; ++i)
#pragma unroll
          for (int j = 0; j <= i; ++j) s.u.fac.Dfac[i * 6 + j] = Dm[i * 6 + j];
#pragma unroll
        for (int i = 0; i < 6; ++i) s.u.fac.Dinv[i] = Dinv[i];
      }
    } else {
      // smooth solve, free joint: L L' qdd = x_base - S_base.pA_1 (reference: src/aba_factor.cuh:139-155)
      float S3[3][3];   // S3[k][i] = S_base rotation k, component i = R1 column k
#pragma unroll
      for (int k = 0; k < 3; ++k)
#pragma unroll
        for (int i = 0; i < 3; ++i) S3[k][i] = R1.m[3 * i + k];
      float qdd[6];
#pragma unroll
      for (int k = 0; k < 6; ++k) qdd[k] = xb[k] - sbase_dot(k, S3[k < 3 ? 0 : k - 3], pA1);
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        float a = qdd[i];
#pragma unroll
        for (int k = 0; k < i; ++k) a = fmaf_(-Dm[i * 6 + k], qdd[k], a);
        qdd[i] = div_rn(a, Dm[i * 6 + i], Dinv[i]);
      }
#pragma unroll
      for (int i = 5; i >= 0; --i) {
        float a = qdd[i];
#pragma unroll
        for (int k = i + 1; k < 6; ++k) a = fmaf_(-Dm[k * 6 + i], qdd[k], a);
        qdd[i] = div_rn(a, Dm[i * 6 + i], Dinv[i]);
      }
#pragma unroll
      for (int k = 0; k < 6; ++k) qb[k] = qdd[k];
#pragma unroll
      for (int i = 0; i < 6; ++i) a6[i] = sbase_col(i, S3, qdd);
    }
  }
  // ---------------- smooth solve root -> leaf (reference: src/aba_factor.cuh:156-164)
  // In the factor's chain layout: the four chains walk root -> leaf in lock-step over depth, every
  // lane of a chain carrying the whole 6-vector acceleration (the per-body operations of the
  // lane-per-body form, redundantly on the chain's lanes), so a level has no cross-lane exchange;
  // the chains start from the pelvis' acceleration (on every lane), the right arm from the torso
  // (chain 2, depth 4).
  // A chain's values outside its depth range are never stored, and the right arm's are replaced
  // at its first level. Each level's LDS operands are read one level ahead.
  if (ncon_max == 0) {
    float a[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) a[k] = a6[k];
    float U[6], S[6], us, iD;
    auto ld = [&](int r) {
      const int b = chain_body(r);
#pragma unroll
      for (int k = 0; k < 6; ++k) { U[k] = s.u.fac.U[b][k]; S[k] = s.u.fac.S[b + 4][k]; }
      us = s.u.fac.U[b][kUs];
      iD = s.u.fac.U[b][kInvD];
    };
    ld(2);
#pragma unroll
    for (int r = 2; r <= kMaxDepth; ++r) {
      if (r == kTorsoDepth + 1) {
        float at[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) at[k] = from_prev_chain(a[k]);   // chain 2's lanes (row_shr:8)
        if (grp == 3) {
#pragma unroll
          for (int k = 0; k < 6; ++k) a[k] = at[k];
        }
      }
      const float Uc[6] = {U[0], U[1], U[2], U[3], U[4], U[5]};
      const float Sc[6] = {S[0], S[1], S[2], S[3], S[4], S[5]};
      const float usc = us, iDc = iD;
      if (r < kMaxDepth) ld(r + 1);
      const float q = (usc - dot6(Uc, a)) * iDc;
#pragma unroll
      for (int k = 0; k < 6; ++k) a[k] = fmaf_(Sc[k], q, a[k]);
      if (r >= c_lo && r <= c_hi && crow == 0) s.Mm[0][chain_body(r) + 4] = q;
    }
  }

  __builtin_amdgcn_s_setprio(3);   // the contact pipeline (see the factor above)
  // ---------------- PASS 1: basis rows, R, aref (reference: src/env_qacc.cuh:67-136)
  const float mu = P.mu;
  static_assert(kContactDofs == 12 && 2 * kContactDofs <= kGroup, "two contacts' rows per pass");
  if (ncon_max > 0) {
    // the basis rows, lane-parallel: in pass ps lane l < 24 forms the three entries of contact
    // 2 ps + l / 12 on its ancestor dof k = l mod 12, walked foot -> root: leg hinges (foot first),
    // then the free base 0..5. Point Jacobian column w x r + lv; on the free base the structural
    // zeros of S_base are skipped (see sbase_dot): translation a gives e_a, rotation a gives w x r.
    const int k = l % kContactDofs;
#pragma unroll
    for (int ps = 0; ps < (kNFoot + 1) / 2; ++ps) {
      if (2 * ps >= ncon_max) break;
      const int ci = 2 * ps + l / kContactDofs;
      const bool on = l < 2 * kContactDofs && ci < ncon;
      const int c = on ? ci : 0;
      const int a = (k < 6) ? (s.con_leg[c] ? 12 : 6) + 5 - k : k - 6;
      const V3 r = vsub(V3{s.con[c][0], s.con[c][1], s.con[c][2]}, p);
      const float* Sa = s.u.fac.S[a];   // (base translation rows: never stored, unused)
      const V3 cr = cross(V3{Sa[0], Sa[1], Sa[2]}, r);
      const V3 leg = vadd(cr, V3{Sa[3], Sa[4], Sa[5]});
      const bool trans = k >= 6 && a < 3;
      const V3 jc{k < 6 ? leg.x : (trans ? (a == 0 ? 1.f : 0.f) : cr.x),
                  k < 6 ? leg.y : (trans ? (a == 1 ? 1.f : 0.f) : cr.y),
                  k < 6 ? leg.z : (trans ? (a == 2 ? 1.f : 0.f) : cr.z)};
      if (on) { s.Eb[c][0][k] = jc.z; s.Eb[c][1][k] = mu * jc.y; s.Eb[c][2][k] = -mu * jc.x; }
    }
  }
  wave_sync();   // the basis rows in LDS
  if (ncon_max > 0 && l < ncon) {
    const int c = l;
    const int legbase = s.con_leg[c] ? 12 : 6;
    // the reference velocities of the four pyramid rows: sum_k e_a[k] qd[k] in dof order
    float v0 = 0.f, v1 = 0.f, v2 = 0.f;
#pragma unroll
    for (int k = 0; k < kContactDofs; ++k) {
      const float qd = s.qvel[(k < 6) ? legbase + 5 - k : k - 6];
      v0 = fmaf_(s.Eb[c][0][k], qd, v0); v1 = fmaf_(s.Eb[c][1][k], qd, v1); v2 = fmaf_(s.Eb[c][2][k], qd, v2);
    }
    const float dmax = MF::foot_solimp[1], tc = MF::foot_solref[0], dr = MF::foot_solref[1];
    const float bcoef = 2.f / (dmax * tc);
    const float kcoef = 1.f / (dmax * dmax * tc * tc * dr * dr);
    const float pyr = (1.f + mu * mu) * (2.f * mu * mu / MF::foot_impratio);
    const float pen = s.con[c][3], imp = foot_impedance(pen);
    s.Rc[c] = div_rn(s.con_w0[c] * pyr * (1.f - imp), imp, rcp_rn(imp));
    const float kip = kcoef * imp * pen;
    s.aref[4 * c + 0] = -bcoef * (v0 + v1) - kip;
    s.aref[4 * c + 1] = -bcoef * (v0 - v1) - kip;
    s.aref[4 * c + 2] = -bcoef * (v0 + v2) - kip;
    s.aref[4 * c + 3] = -bcoef * (v0 - v2) - kip;
  }
  wave_sync();

  // ---------------- PASS 2: M^-1 solves, lane j = basis column j (reference: src/aba_factor.cuh:121-165,
  // src/env_qacc.cuh:137-152). Lane 0 finishes column 0, the smooth solve: its leaf -> root part
  // (pA_1, u) came with the factor, its base and root -> leaf parts are the code below with
  // x_base, pA_1 and u from the smooth solve.
  // The traversal is unrolled over the static tree. Articulated bias forces travel as explicit
  // carries along each chain (arm chains end in the torso 16, leg and waist chains in the pelvis 1);
  // parents with several children accumulate them in the reference's descending-child order.
  float xb0[6];   // the smooth right-hand side on the base dofs (lane 1 holds it)
  if (ncon_max > 0) {
#pragma unroll
    for (int k = 0; k < 6; ++k) xb0[k] = xb[k];
  }
  if (ncon_max > 0 && ncon_max <= kChainSolveCon) {
    // Chain layout (waves with at most two contacts per world, at most seven columns): lane
    // (g, c) = (l / 8, l mod 8) takes column c (0: smooth, 1 + 3 c' + a: basis row a of contact
    // c'; c = 7 idle) on chain g of the factor's layout. The same operations per column and body
    // as the lane-per-column form below, but the four chains walk in lock-step over depth: 6 + 10
    // levels instead of 12 + 29 bodies in sequence.
    const int col = l & 7;
    const int cj = col >= 1 ? (col - 1) / 3 : 0, aj = col >= 1 ? (col - 1) % 3 : 0;
    const bool basis = col >= 1 && col < 7 && cj < ncon;
    const bool right = s.con_leg[cj] != 0;
    const float* eb = s.Eb[cj][aj];
    const bool smooth = col == 0;
    const bool wr = col < 7;
    // leaf -> root over the legs (the waist/arm subtree carries zero bias for the basis rows, as
    // below): the lanes of chains 0 and 2 walk the left leg 7..2, those of 1 and 3 the right leg
    // 13..8 (chains 2 and 3 repeat 0 and 1), body = depth + loff; operands read a level ahead
    const int lc = grp & 1, loff = lc ? 6 : 0;
    const bool own = basis && (lc ? right : !right);
    float ul[6];                 // u of the lane's leg bodies at depth 2..7
    float car[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    {
      const float* const pS = &s.u.fac.S[loff + 4][0];
      const float* const pU = &s.u.fac.U[loff][0];
      const float* const pD = &s.u.fac.U[loff][kInvD];
      float nS[6], nU[6], nD, nE;
      auto ld = [&](int d) {
#pragma unroll
        for (int k = 0; k < 6; ++k) { nS[k] = pS[kRow * d + k]; nU[k] = pU[kRow * d + k]; }
        nD = pD[kRow * d];
        nE = eb[7 - d];   // xrhs(d + loff + 4) before its select (both legs: entry 7 - d)
      };
      ld(7);
#pragma unroll
      for (int d = 7; d >= 2; --d) {
        float Sd[6], Ud[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) { Sd[k] = nS[k]; Ud[k] = nU[k]; }
        const float iD = nD, e = nE;
        if (d > 2) ld(d - 1);
        float pb[6];   // the leaf (7, 13) has no child
#pragma unroll
        for (int k = 0; k < 6; ++k) pb[k] = d == 7 ? 0.f : car[k];
        const float ub = (own ? e : 0.f) - dot6(Sd, pb);
        ul[d - 2] = ub;
        const float ud = ub * iD;
#pragma unroll
        for (int k = 0; k < 6; ++k) car[k] = fmaf_(Ud[k], ud, pb[k]);
      }
    }
    // pelvis: p1 = c8 + c2 (the right leg's root first) on chain 0's lanes, then to every chain
    float p1[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const float c8 = from_next_chain(car[k]);
      float v = smooth ? pAs[k] : c8 + car[k];
      const float v1 = from_prev_chain(v);           // chain 0 -> 1
      v = grp == 1 ? v1 : v;
      const float v2 = from_lower_row(v);            // chains 0, 1 -> 2, 3
      p1[k] = grp >= 2 ? v2 : v;
    }
    float qdd[6], a1[6], xbj[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) xbj[k] = smooth ? xb0[k] : (basis ? eb[6 + k] : 0.f);
    base_solve(s, xbj, p1, qdd, a1);
    float* const ycol = s.Mm[wr ? col : 0];
    if (grp == 0 && wr) {
#pragma unroll
      for (int k = 0; k < 6; ++k) ycol[k] = qdd[k];
    }
    // root -> leaf, the chains in lock-step: legs and waist from the pelvis at depth 2, the right
    // arm from the torso (chain 2's depth-4 result) at depth 5
    {
      const float* const pS = &s.u.fac.S[c_off + 4][0];
      const float* const pU = &s.u.fac.U[c_off][0];
      const float* const pD = &s.u.fac.U[c_off][kInvD];
      const float* const pUs = &s.u.fac.U[c_off][kUs];
      float nS[6], nU[6], nD, nUs;
      auto ld = [&](int d) {
#pragma unroll
        for (int k = 0; k < 6; ++k) { nS[k] = pS[kRow * d + k]; nU[k] = pU[kRow * d + k]; }
        nD = pD[kRow * d];
        nUs = pUs[kRow * d];
      };
      ld(2);
      float ac[6];
#pragma unroll
      for (int k = 0; k < 6; ++k) ac[k] = a1[k];
#pragma unroll
      for (int d = 2; d <= kMaxDepth; ++d) {
        if (d == kTorsoDepth + 1) {
#pragma unroll
          for (int k = 0; k < 6; ++k) {
            const float at = from_prev_chain(ac[k]);   // chain 2 -> 3
            ac[k] = grp == 3 ? at : ac[k];
          }
        }
        float Sd[6], Ud[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) { Sd[k] = nS[k]; Ud[k] = nU[k]; }
        const float iD = nD, us = nUs;
        if (d < kMaxDepth) ld(d + 1);
        const float ub = smooth ? us : ((grp <= 1 && d <= 7) ? ul[d <= 7 ? d - 2 : 0] : 0.f);
        const float q = (ub - dot6(Ud, ac)) * iD;
        if (wr && d >= c_lo && d <= c_hi) ycol[chain_body(d) + 4] = q;
#pragma unroll
        for (int k = 0; k < 6; ++k) ac[k] = fmaf_(Sd[k], q, ac[k]);
      }
    }
  } else if (ncon_max > 0) {
    const int j = l;
    const int cj = (j >= 1 && j < kCols) ? (j - 1) / 3 : 0, aj = (j >= 1) ? (j - 1) % 3 : 0;
    const bool basis = (j >= 1) && (j < kCols) && (cj < ncon);
    const bool right = s.con_leg[cj] != 0;
    const float* eb = s.Eb[cj][aj];
    // right-hand side entry of dof d, read on demand: the contact basis row e_{c,a} on its 12
    // ancestor dofs, 0 elsewhere and for idle lanes
    auto xrhs = [&](int d) -> float {
      if (d < 6) return basis ? eb[6 + d] : 0.f;
      if (d < 12) return (basis && !right) ? eb[11 - d] : 0.f;
      if (d < 18) return (basis && right) ? eb[17 - d] : 0.f;
      return 0.f;
    };
    // leaf -> root. The basis right-hand sides live on the base and leg dofs (the feet hang off
    // bodies 7 and 13, legs 2..13), so the waist/arm subtree (bodies 14..30) carries zero
    // articulated bias: u = 0 - S.0 = +0 and its contribution to the pelvis is +0; skipping it
    // changes no bit. The two legs are independent chains and are walked interleaved (right leg
    // 13..8 with left leg 7..2) so their dependency chains overlap; the pelvis then adds the
    // right leg's root (8) before the left leg's (2), the reference's descending order.
    static_assert(foot_body[0] < 14 && foot_body[kNFoot - 1] < 14 && body_parent[14] == 1, "leg layout");
    static_assert(body_parent[2] == 1 && body_parent[8] == 1 && body_nchild[7] == 0 && body_nchild[13] == 0, "legs");
    float u[kNBody];
#pragma unroll
    for (int b = 14; b < kNBody; ++b) u[b] = 0.f;
    // Each body's LDS operands are read one body ahead (`nxt`) so their latency overlaps the
    // current body's arithmetic; the pin keeps the reads from running further ahead.
    // (only plain loads: a value used before the pin would make it wait for them)
    struct UpIn { float S[6], U[6], iD, e; };
    auto ld_up = [&](int b, UpIn& f) {
#pragma unroll
      for (int k = 0; k < 6; ++k) { f.S[k] = s.u.fac.S[b + 4][k]; f.U[k] = s.u.fac.U[b][k]; }
      f.iD = s.u.fac.U[b][kInvD];
      f.e = eb[b < 8 ? 7 - b : 13 - b];   // xrhs(b + 4) before its select
    };
    constexpr int kUpOrder[12] = {13, 7, 12, 6, 11, 5, 10, 4, 9, 3, 8, 2};
    float car[2][6] = {}, croot[2][6];   // [0] right leg (13..8), [1] left leg (7..2)
    UpIn cur, nxt;
    ld_up(kUpOrder[0], cur);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      const int b = kUpOrder[i], g = i & 1;
      if (i + 1 < 12) ld_up(kUpOrder[i + 1], nxt);
      float pb[6];
#pragma unroll
      for (int k = 0; k < 6; ++k) pb[k] = body_nchild[b] == 0 ? 0.f : car[g][k];
      const bool own = basis && (b < 8 ? !right : right);
      const float ub = (own ? cur.e : 0.f) - dot6(cur.S, pb);
      u[b] = ub;
      const float ud = ub * cur.iD;
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const float c = fmaf_(cur.U[k], ud, pb[k]);
        if (body_parent[b] == 1) croot[g][k] = c;
        else car[g][k] = c;
      }
      G1_PIN6(car[g]);
      __asm__ volatile("" : "+v"(u[b]));
      if (i + 1 < 12) cur = nxt;
    }
    const float (&c8)[6] = croot[0];
    const float (&c2)[6] = croot[1];
    float p1[6];
    const bool smooth = j == 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) p1[k] = smooth ? pAs[k] : c8[k] + c2[k];
    // free joint: D qdd = x_base - S_base.pA_1 with D = L L'
    float qdd[6], a1[6], xbj[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) xbj[k] = smooth ? xb0[k] : xrhs(k);
    base_solve(s, xbj, p1, qdd, a1);
    float* ycol = s.Mm[j < kCols ? j : kCols - 1];
    const bool wr = j < kCols;
    if (wr) {
#pragma unroll
      for (int k = 0; k < 6; ++k) ycol[k] = qdd[k];
    }
    G1_PIN6(a1);
    // root -> leaf over five independent chains, walked interleaved: legs and waist from the
    // pelvis (2.., 8.., 14..16), then both arms from the torso (17.., 24..); operands read one
    // body ahead as in the leaf -> root pass
    static_assert(body_parent[14] == 1 && body_parent[17] == 16 && body_parent[24] == 16, "chains");
    struct DnIn { float U[6], S[6], iD, us; };
    auto ld_dn = [&](int b, DnIn& f) {
#pragma unroll
      for (int k = 0; k < 6; ++k) { f.U[k] = s.u.fac.U[b][k]; f.S[k] = s.u.fac.S[b + 4][k]; }
      f.iD = s.u.fac.U[b][kInvD];
      f.us = s.u.fac.U[b][kUs];
    };
    constexpr int kDownOrder[29] = {2, 8, 14, 3, 9, 15, 4, 10, 16, 5, 11, 6, 12, 7, 13,
                                    17, 24, 18, 25, 19, 26, 20, 27, 21, 28, 22, 29, 23, 30};
    float acc[5][6];   // left leg, right leg, waist (the torso 16 at its end), left arm, right arm
    DnIn dc, dn;
    ld_dn(kDownOrder[0], dc);
#pragma unroll
    for (int i = 0; i < 29; ++i) {
      const int b = kDownOrder[i];
      const int ch = b < 8 ? 0 : b < 14 ? 1 : b < 17 ? 2 : b < 24 ? 3 : 4;
      if (i + 1 < 29) ld_dn(kDownOrder[i + 1], dn);
      float ap[6];
#pragma unroll
      for (int k = 0; k < 6; ++k) ap[k] = body_parent[b] == 1 ? a1[k] : body_parent[b] == 16 ? acc[2][k] : acc[ch][k];
      const float q = ((smooth ? dc.us : u[b]) - dot6(dc.U, ap)) * dc.iD;
      if (wr) ycol[b + 4] = q;
#pragma unroll
      for (int k = 0; k < 6; ++k) acc[ch][k] = fmaf_(dc.S[k], q, ap[k]);
      G1_PIN6(acc[ch]);
      if (i + 1 < 29) dc = dn;
    }
  }
  wave_sync();

  if (ncon_max == 0) {
#pragma unroll
    for (int k = 0; k < 6; ++k) bqacc[k] = qb[k];   // every lane: each integrates the free joint
    jqacc = L.hinge ? s.Mm[0][L.b + 4] : 0.f;
    __builtin_amdgcn_s_setprio(0);
    wave_sync();
    return ncon;
  }

  // ---------------- Gram blocks + b (reference: src/env_qacc.cuh:154-192); G aliases the factor
  // Block row c of column j: g_a = e_{c,a} . m_j over contact c's 12 ancestor dofs (dof
  // legbase + 5 - k on the leg, legbase 6 left, 12 right; k - 6 on the base), and b_c from the same
  // products with the smooth column (j = 0).
  if (ncon_max <= kChainSolveCon) {
    // lane (c, j) = (l / 8, l mod 8): one block row per lane (contact c <= 1, column j <= 6); the
    // lanes of column 0 form b of their contact
    const int c = l >> 3, j = l & 7;
    const int cp = j >= 1 ? (j - 1) / 3 : 0, bcol = j >= 1 ? (j - 1) % 3 : 0;
    const bool blk = j >= 1 && j < 7 && cp < ncon && c <= cp;
    const bool bvc = j == 0 && c < ncon;
    const int cc = c < kChainSolveCon ? c : 0;
    const float* mcol = s.Mm[j < 7 ? j : 0];
    const bool rightleg = s.con_leg[cc] != 0;
    float g0 = 0.f, g1 = 0.f, g2 = 0.f;
#pragma unroll
    for (int k = 0; k < kContactDofs; ++k) {
      const float mv = (k < 6) ? (rightleg ? mcol[17 - k] : mcol[11 - k]) : mcol[k - 6];
      g0 = fmaf_(s.Eb[cc][0][k], mv, g0); g1 = fmaf_(s.Eb[cc][1][k], mv, g1); g2 = fmaf_(s.Eb[cc][2][k], mv, g2);
    }
    if (blk) {
      const int pr = cp * (cp + 1) / 2 + c;
      s.u.G[pr][0 * 3 + bcol] = g0; s.u.G[pr][1 * 3 + bcol] = g1; s.u.G[pr][2 * 3 + bcol] = g2;
    }
    if (bvc) {
      s.bvec[4 * c + 0] = fmaf_(0.f, g2, fmaf_(1.f, g1, 1.f * g0)) - s.aref[4 * c + 0];
      s.bvec[4 * c + 1] = fmaf_(0.f, g2, fmaf_(-1.f, g1, 1.f * g0)) - s.aref[4 * c + 1];
      s.bvec[4 * c + 2] = fmaf_(1.f, g2, fmaf_(0.f, g1, 1.f * g0)) - s.aref[4 * c + 2];
      s.bvec[4 * c + 3] = fmaf_(-1.f, g2, fmaf_(0.f, g1, 1.f * g0)) - s.aref[4 * c + 3];
    }
    wave_sync();
  } else {
    float bb0 = 0.f, bb1 = 0.f, bb2 = 0.f;
    if (l < ncon) {
      const int legbase = s.con_leg[l] ? 12 : 6;
#pragma unroll
      for (int k = 0; k < kContactDofs; ++k) {
        const int a = (k < 6) ? legbase + 5 - k : k - 6;
        const float qa = s.Mm[0][a];
        bb0 = fmaf_(s.Eb[l][0][k], qa, bb0); bb1 = fmaf_(s.Eb[l][1][k], qa, bb1); bb2 = fmaf_(s.Eb[l][2][k], qa, bb2);
      }
    }
    wave_sync();   // factor region is dead from here on: the Gram blocks overwrite it
    {
      const int j = l;
      const int cp = (j >= 1) ? (j - 1) / 3 : 0, bcol = (j >= 1) ? (j - 1) % 3 : 0;
      const bool active = (j >= 1) && (cp < ncon);
      // the lane's solve column on the base and both legs' dofs (0..17), read once for all c
      float mj[18];
      const float* mcol = s.Mm[active ? j : 0];
#pragma unroll
      for (int a = 0; a < 18; ++a) mj[a] = mcol[a];
#pragma unroll
      for (int c = 0; c < kNFoot; ++c) {
        if (c >= ncon_max) break;
        if (active && c <= cp) {
          const bool rightleg = s.con_leg[c] != 0;
          float g0 = 0.f, g1 = 0.f, g2 = 0.f;
#pragma unroll
          for (int k = 0; k < kContactDofs; ++k) {
            // dof a = legbase + 5 - k on the leg (legbase 6 left, 12 right), k - 6 on the base
            const float mv = (k < 6) ? (rightleg ? mj[17 - k] : mj[11 - k]) : mj[k - 6];
            g0 = fmaf_(s.Eb[c][0][k], mv, g0); g1 = fmaf_(s.Eb[c][1][k], mv, g1); g2 = fmaf_(s.Eb[c][2][k], mv, g2);
          }
          const int pr = cp * (cp + 1) / 2 + c;
          s.u.G[pr][0 * 3 + bcol] = g0; s.u.G[pr][1 * 3 + bcol] = g1; s.u.G[pr][2 * 3 + bcol] = g2;
        }
      }
    }
    if (l < ncon) {
      s.bvec[4 * l + 0] = fmaf_(0.f, bb2, fmaf_(1.f, bb1, 1.f * bb0)) - s.aref[4 * l + 0];
      s.bvec[4 * l + 1] = fmaf_(0.f, bb2, fmaf_(-1.f, bb1, 1.f * bb0)) - s.aref[4 * l + 1];
      s.bvec[4 * l + 2] = fmaf_(1.f, bb2, fmaf_(0.f, bb1, 1.f * bb0)) - s.aref[4 * l + 2];
      s.bvec[4 * l + 3] = fmaf_(-1.f, bb2, fmaf_(0.f, bb1, 1.f * bb0)) - s.aref[4 * l + 3];
    }
    wave_sync();
  }

  // ---------------- A column of row-lane i (reference: src/env_qacc.cuh:154-190); pyramid
  // directions d0=(1,1,0) d1=(1,-1,0) d2=(1,0,1) d3=(1,0,-1). For a pair c < c' the reference
  // expands d_k' G[c][c'] d_k'' once and mirrors it; within one contact it keeps the value
  // computed with (k, k') = (larger, smaller).
  const int nefc = 4 * ncon, nefc_max = 4 * ncon_max;
  const int ci = l >> 2, ki = l & 3;
  const bool row = l < nefc;
  auto dcoef = [](int k, int a) -> float {
    return a == 0 ? 1.f : (a == 1 ? (k == 0 ? 1.f : (k == 1 ? -1.f : 0.f)) : (k == 2 ? 1.f : (k == 3 ? -1.f : 0.f)));
  };
  // Entries are formed by every lane (branch-free; the G block and R indices stay inside their
  // arrays for every lane) and kept where (row, column) is a constraint pair; the row loop stops at
  // the wave's largest row count.
  float Acol[kMaxEfc];
#pragma unroll
  for (int ii = 0; ii < kMaxEfc; ++ii) Acol[ii] = 0.f;
  float Aii = 1.f;   // the lane's diagonal entry, taken as it is formed (1 on lanes without a row)
  const float Rci = s.Rc[ci];
  // pyramid coefficients of the lane's own row (d0 = 1 for every direction)
  const float dki1 = dcoef(ki, 1), dki2 = dcoef(ki, 2);
#pragma unroll
  for (int c2 = 0; c2 < kNFoot; ++c2) {
    if (c2 >= ncon_max) continue;
    const int lo = c2 < ci ? c2 : ci, hi = c2 < ci ? ci : c2;
    const float* Gp = s.u.G[hi * (hi + 1) / 2 + lo];
    float G[9];
#pragma unroll
    for (int e = 0; e < 9; ++e) G[e] = Gp[e];
    const bool lt = c2 < ci, eq = c2 == ci, keep = row && c2 < ncon;
#pragma unroll
    for (int k2 = 0; k2 < 4; ++k2) {
      // (klo, khi) = (k2, ki) if c2 < ci, (ki, k2) if c2 > ci, (max, min) within one contact
      const bool k2lo = lt || (eq && k2 >= ki);
      const float dk1 = dcoef(k2, 1), dk2 = dcoef(k2, 2);
      const float dl1 = k2lo ? dk1 : dki1, dl2 = k2lo ? dk2 : dki2;
      const float dh1 = k2lo ? dki1 : dk1, dh2 = k2lo ? dki2 : dk2;
      const float t0 = fmaf_(dl2, G[6], fmaf_(dl1, G[3], 1.f * G[0]));
      const float t1 = fmaf_(dl2, G[7], fmaf_(dl1, G[4], 1.f * G[1]));
      const float t2 = fmaf_(dl2, G[8], fmaf_(dl1, G[5], 1.f * G[2]));
      float val = fmaf_(t2, dh2, fmaf_(t1, dh1, t0 * 1.f));
      const bool diag = eq && k2 == ki;
      val = diag ? val + Rci : val;
      Acol[4 * c2 + k2] = (keep && !diag) ? val : 0.f;   // the diagonal is held apart (Aii)
      Aii = (diag && row) ? val : Aii;
    }
  }
  const float bi = row ? s.bvec[l] : 0.f;

  // ---------------- projected Gauss-Seidel (reference: src/contact.cuh:159-171), P.pgs sweeps, in
  // the row-scaled residual form of pgs_sweep. A sweep that leaves every f of a world bit-for-bit
  // unchanged ends that world's solve: without a fresh residual in between, every later sweep would
  // repeat it exactly (its changes are all +0), and the world takes no fresh residual after it; the
  // wave stops once both worlds are done.
  float fi = 0.f;
  const float yi = rcp_rn(Aii);
  const float cb = bi * yi;
  float ri = cb;
  auto solve = [&](auto wc) {
    constexpr int W = decltype(wc)::value;
#pragma unroll
    for (int ii = 0; ii < W; ++ii) Acol[ii] = Acol[ii] * yi;
    bool done = false;   // this world's solve has ended
#pragma unroll 1
    for (int it = 0; it < P.pgs; ++it) {
      if (it > 0 && it % kPgsRefresh == 0) {
        // fresh residuals: every lane reads every f of its world
        s.f[l] = fi;
        wave_sync();
        float t = cb;
#pragma unroll
        for (int k = 0; k < W; ++k)
          if (k < nefc_max) t = fmaf_(Acol[k], s.f[k], t);
        wave_sync();
        ri = done ? ri : t;
      }
      const float f0 = fi;
      unsigned long long lanes0 = kPgsLanes0;
      __asm__ volatile("" : "+s"(lanes0));
      pgs_sweep<0, W>(Acol, l, lanes0, nefc_max, fi, ri);
      const unsigned long long m = __ballot(__float_as_uint(fi) != __float_as_uint(f0));
      if (m == 0ull) break;
      done = done || ((unsigned)(m >> (32 * group_id())) == 0u);
    }
  };
  // up to 32 rows: the paired-row form of pgs_sweep_pair (lane l: rows l mod 16 and 16 + l mod 16)
  auto solve_pairs = [&]() {
#pragma unroll
    for (int ii = 0; ii < kMaxEfc; ++ii) Acol[ii] = Acol[ii] * yi;
    // A v_permlane16_swap of a value with itself gives every lane of a group the value of lane
    // l mod 16 of the group's first 16-lane row (first result) and of its second row (second).
    auto split = [](float v, float& lo, float& hi) {
      const auto pq = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      lo = __uint_as_float(pq[0]);
      hi = __uint_as_float(pq[1]);
    };
    float Pr[kMaxEfc], Qr[kMaxEfc];   // entries (lo, k) and (hi, k) of the scaled A
#pragma unroll
    for (int k = 0; k < kMaxEfc; ++k) {
      if (k % 4 == 0 && k >= nefc_max) break;   // rows past nefc_max are never read
      split(Acol[k], Pr[k], Qr[k]);
    }
    float clo, chi;
    split(cb, clo, chi);
    float flo = 0.f, fhi = 0.f, rlo = clo, rhi = chi;
    bool done = false;   // this world's solve has ended
#pragma unroll 1
    for (int it = 0; it < P.pgs; ++it) {
      if (it > 0 && it % kPgsRefresh == 0) {
        // fresh residuals: every lane reads every f of its world (row l from lane l's copy)
        s.f[l] = l < kGroup / 2 ? flo : fhi;
        wave_sync();
        float tlo = clo, thi = chi;
#pragma unroll
        for (int k = 0; k < kMaxEfc; ++k)
          if (k < nefc_max) {
            const float fk = s.f[k];
            tlo = fmaf_(Pr[k], fk, tlo);
            thi = fmaf_(Qr[k], fk, thi);
          }
        wave_sync();
        rlo = done ? rlo : tlo;
        rhi = done ? rhi : thi;
      }
      const float flo0 = flo, fhi0 = fhi;
      unsigned long long lanes0 = kPgsLanes0;
      __asm__ volatile("" : "+s"(lanes0));
      pgs_sweep_pair<0>(Pr, Qr, lanes0, nefc_max, flo, fhi, rlo, rhi);
      const unsigned long long m = __ballot(__float_as_uint(flo) != __float_as_uint(flo0) ||
                                            __float_as_uint(fhi) != __float_as_uint(fhi0));
      if (m == 0ull) break;
      done = done || ((unsigned)(m >> (32 * group_id())) == 0u);
    }
    fi = l < kGroup / 2 ? flo : fhi;   // row l
  };
  if (nefc_max <= 4) solve(std::integral_constant<int, 4>());
  else if (nefc_max <= kGroup / 2) solve(std::integral_constant<int, kGroup / 2>());
  else solve_pairs();
  __builtin_amdgcn_s_setprio(0);
  if (row) s.f[l] = fi;
  wave_sync();

  // ---------------- qacc = qacc_smooth + sum_c sum_a fb_c[a] m_{c,a} (reference: src/env_qacc.cuh:196-211)
  // lane l: dof l and (lanes 0..2) dof 32 + l, both accumulated in one pass over the contacts
  {
    static_assert(kNV <= 2 * kGroup, "two dofs per lane");
    const int d1 = l, d2 = kGroup + l < kNV ? kGroup + l : l;
    float dq1 = 0.f, dq2 = 0.f;
    const float s1 = s.Mm[0][d1], s2 = s.Mm[0][d2];
    // Contact c's four forces and its three solve columns at the lane's dofs, read one contact
    // ahead (every index stays inside f and Mm), so that the next contact's reads overlap this one's
    // arithmetic instead of each contact waiting on its own reads; a contact the lane's world does
    // not have (c >= ncon) is computed and not added.
    float F[4], M1[3], M2[3];
    auto ld = [&](int c) {
#pragma unroll
      for (int k = 0; k < 4; ++k) F[k] = s.f[4 * c + k];
#pragma unroll
      for (int a = 0; a < 3; ++a) { M1[a] = s.Mm[1 + a + 3 * c][d1]; M2[a] = s.Mm[1 + a + 3 * c][d2]; }
    };
    ld(0);
#pragma unroll
    for (int c = 0; c < kNFoot; ++c) {
      if (c >= ncon_max) break;
      const float f0 = F[0], f1 = F[1], f2 = F[2], f3 = F[3];
      const float m10 = M1[0], m11 = M1[1], m12 = M1[2], m20 = M2[0], m21 = M2[1], m22 = M2[2];
      if (c + 1 < kNFoot) ld(c + 1);
      const float fb0 = f0 + f1 + f2 + f3, fb1 = f0 - f1, fb2 = f2 - f3;
      const float t1 = fmaf_(fb2, m12, fmaf_(fb1, m11, fb0 * m10));
      const float t2 = fmaf_(fb2, m22, fmaf_(fb1, m21, fb0 * m20));
      dq1 = c < ncon ? dq1 + t1 : dq1;
      dq2 = c < ncon ? dq2 + t2 : dq2;
    }
    s.qacc[d1] = s1 + dq1;
    if (kGroup + l < kNV) s.qacc[d2] = s2 + dq2;
  }
  wave_sync();
#pragma unroll
  for (int k = 0; k < 6; ++k) bqacc[k] = s.qacc[k];   // every lane: each integrates the free joint
  jqacc = L.hinge ? s.qacc[L.b + 4] : 0.f;
  wave_sync();
  return ncon;
}

// ================================================================ Euler + position integration
// v += dt qacc with the reference's NaN/clamp guard (src/g1_env.cu:154-160), then q += dt v,
// base quaternion q <- normalize(q (x) exp(w dt)) (src/dynamics.cuh:333-355).
__device__ __forceinline__ void integrate_lane(const LaneModel& L, LaneState& st, const float (&bqacc)[6], float jqacc,
                                               bool guard) {
  const float dt = MF::dt;
  auto upd = [&](float v, float a) {
    float n = fmaf_(dt, a, v);
    if (guard) {
      if (!isfinite(n)) n = 0.f;
      if (n > 50.f) n = 50.f; else if (n < -50.f) n = -50.f;
    }
    return n;
  };
  if (L.hinge) {
    st.jqd = upd(st.jqd, jqacc);
    st.jq = fmaf_(dt, st.jqd, st.jq);
  }
  {
    // the free joint on every lane (the same operations on the same values, so every lane holds the
    // pelvis state; lane 1 is the one that stores it)
#pragma unroll
    for (int k = 0; k < 6; ++k) st.bqd[k] = upd(st.bqd[k], bqacc[k]);
    st.bq[0] = fmaf_(dt, st.bqd[0], st.bq[0]); st.bq[1] = fmaf_(dt, st.bqd[1], st.bq[1]);
    st.bq[2] = fmaf_(dt, st.bqd[2], st.bq[2]);
    V3 v{st.bqd[3] * dt, st.bqd[4] * dt, st.bqd[5] * dt};
    const float ang = sqrtf(fmaf_(v.z, v.z, fmaf_(v.y, v.y, v.x * v.x)));
    Q4 dq;
    if (ang < 1e-9f) dq = {1.f, 0.5f * v.x, 0.5f * v.y, 0.5f * v.z};
    else {
      float sh, ch;
      sincos_small_rn(0.5f * ang, sh, ch);
      const float sn = div_rn(sh, ang, rcp_rn(ang));
      dq = {ch, v.x * sn, v.y * sn, v.z * sn};
    }
    Q4 qn = qnorm(qmul(Q4{st.bq[3], st.bq[4], st.bq[5], st.bq[6]}, dq));
    st.bq[3] = qn.w; st.bq[4] = qn.x; st.bq[5] = qn.y; st.bq[6] = qn.z;
  }
}

}  // namespace g1k
