// g1_oracle.cpp -- CPU restatement of the g1.cu fused-rollout algorithm. TEST INFRASTRUCTURE ONLY.
//
// This file is the checker, never the product: only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg load the library built from it. The GPU path (libg1env.so) never
// links, loads or calls it.
//
// Every function restates the reference's arithmetic in the reference's operation order (fp32
// parity is order-sensitive), templated on the scalar type so the same code yields the fp32
// oracle (parity vs the GPU) and the fp64 oracle (parity vs the MuJoCo fixtures). Citations are
// file:line into the reference tree (Infatoshi/g1.cu). Build: oracle/Makefile (-ffp-contract=off:
// the only fused operations are the explicit fma_ calls; -mfma: hardware fma, which returns the
// same correctly rounded results as the library fma on every x86-64 host that has it).
//
// Pinning (tests/test_oracle_*.py): FK/bias/qacc/M against bench/ref_traj.npz (MuJoCo fp64);
// fp32 bias/qacc against bench/cuda_fk.bin and aba_qacc.bin; 300-step smooth trajectories against
// cuda_traj.bin/aba_traj.bin; implicit PD against implicit_ref.npz/implicit_cuda.bin; contact
// qacc against contact_validate.bin (pgs=2000); closed forms (M*solveM(x)=x with dense CRBA,
// multi-RHS == single solves, PGS == NNLS at convergence, MLP == torch, log-prob closed form,
// reward/termination hand cases).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <algorithm>
#include <type_traits>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../g1.cu_amd/csrc/g1_model_tables.h"
#include "../g1.cu_amd/csrc/tree.h"

namespace orc {

using namespace g1;

template <class R> using M = ModelT<R>;

template <class R> struct V3 { R x, y, z; };
template <class R> struct Q4 { R w, x, y, z; };

// Fused multiply-add, the one contraction this restatement uses, always explicit: a sum of
// products a0 b0 + a1 b1 + ... is evaluated left to right as s = a0 b0, s = fma(a_i, b_i, s)
// (a difference as fma(-a_i, b_i, s)); an accumulation s = 0; s += a_i b_i as s = fma(a_i, b_i, s)
// from s = 0; x + a b as fma(a, b, x). Everything else rounds every operation (-ffp-contract=off).
template <class R> static inline R fma_(R a, R b, R c) { return std::fma(a, b, c); }

template <class R> static inline V3<R> vadd(V3<R> a, V3<R> b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
template <class R> static inline V3<R> vsub(V3<R> a, V3<R> b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
template <class R> static inline V3<R> cross(V3<R> a, V3<R> b) {
  return {fma_(-a.z, b.y, a.y * b.z), fma_(-a.x, b.z, a.z * b.x), fma_(-a.y, b.x, a.x * b.y)};
}
template <class R> static inline R dot3(V3<R> a, V3<R> b) { return fma_(a.z, b.z, fma_(a.y, b.y, a.x * b.x)); }

// Hamilton product (reference: src/dynamics.cuh:17-24)
template <class R> static inline Q4<R> qmul(Q4<R> a, Q4<R> b) {
  return {fma_(-a.z, b.z, fma_(-a.y, b.y, fma_(-a.x, b.x, a.w * b.w))),
          fma_(-a.z, b.y, fma_(a.y, b.z, fma_(a.x, b.w, a.w * b.x))),
          fma_(a.z, b.x, fma_(a.y, b.w, fma_(-a.x, b.z, a.w * b.y))),
          fma_(a.z, b.w, fma_(-a.y, b.x, fma_(a.x, b.y, a.w * b.z)))};
}
// v' = v + w t + u x t, t = 2 u x v (reference: src/dynamics.cuh:26-35)
template <class R> static inline V3<R> qrot(Q4<R> q, V3<R> v) {
  V3<R> u{q.x, q.y, q.z};
  V3<R> c = cross(u, v);
  V3<R> t{R(2) * c.x, R(2) * c.y, R(2) * c.z};
  V3<R> ut = cross(u, t);
  return {fma_(q.w, t.x, v.x) + ut.x, fma_(q.w, t.y, v.y) + ut.y, fma_(q.w, t.z, v.z) + ut.z};
}
// fp32 transcendentals are correctly rounded (evaluated in fp64, rounded once), so every
// implementation of the algorithm that does the same yields bit-identical values: the contact
// force is stiff in the foot height and amplifies 1-ulp differences in FK rotations.
template <class R> static inline R sin_(R x) { return R(std::sin(double(x))); }
template <class R> static inline R cos_(R x) { return R(std::cos(double(x))); }
template <class R> static inline R pow_(R x, R y) { return R(std::pow(double(x), double(y))); }
template <class R> static inline R sqrt_(R x) { return std::sqrt(x); }
template <class R> static inline R rsqrt_(R x) { return R(1) / sqrt_(x); }
template <class R> static inline R fabs_(R x) { return std::fabs(x); }
template <class R> static inline bool isfinite_(R x) { return std::isfinite(x); }
template <class R> static inline R tanh_(R x) { return std::tanh(x); }
template <class R> static inline R expm1_(R x) { return std::expm1(x); }
template <class R> static inline R exp_(R x) { return std::exp(x); }
// Precision of the forward-kinematics compositions (fk below); a customisation point for the
// operation-counting instantiation (flop_count.cpp), which counts them as its own scalar type.
template <class R> struct ComposePrec { using type = double; };
// Whether fk composes the transforms already in the world frame with the world body's identity (the
// GPU's branch-free form; the same values up to the sign of an exact zero). The counting
// instantiation leaves them out: they move no transform and are not part of the algorithm's work.
template <class R> struct FkComposeIdentity { static constexpr bool value = true; };
// (reference: src/dynamics.cuh:36-39)
template <class R> static inline Q4<R> qnorm(Q4<R> q) {
  R n = rsqrt_(fma_(q.z, q.z, fma_(q.y, q.y, fma_(q.x, q.x, q.w * q.w))));
  return {q.w * n, q.x * n, q.y * n, q.z * n};
}
// (reference: src/dynamics.cuh:40-43)
template <class R> static inline Q4<R> axisangle(V3<R> a, R ang) {
  R h = R(0.5) * ang, s = sin_(h);
  return {cos_(h), a.x * s, a.y * s, a.z * s};
}

template <class R> struct M3 { R m[9]; };
// (reference: src/dynamics.cuh:99-106)
template <class R> static inline M3<R> quat2mat(Q4<R> q) {
  R w = q.w, x = q.x, y = q.y, z = q.z;
  M3<R> r;
  // 1 - 2 s is fma(-2, s, 1) exactly (2 s is exact)
  r.m[0] = fma_(R(-2), fma_(z, z, y * y), R(1)); r.m[1] = 2 * fma_(-w, z, x * y); r.m[2] = 2 * fma_(w, y, x * z);
  r.m[3] = 2 * fma_(w, z, x * y); r.m[4] = fma_(R(-2), fma_(z, z, x * x), R(1)); r.m[5] = 2 * fma_(-w, x, y * z);
  r.m[6] = 2 * fma_(-w, y, x * z); r.m[7] = 2 * fma_(w, x, y * z); r.m[8] = fma_(R(-2), fma_(y, y, x * x), R(1));
  return r;
}
// R diag(d) R^T (reference: src/dynamics.cuh:109-115)
template <class R> static inline M3<R> world_inertia(const M3<R>& Rm, V3<R> d) {
  M3<R> o;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j)
      o.m[3 * i + j] = fma_(Rm.m[3 * i + 2] * d.z, Rm.m[3 * j + 2],
                            fma_(Rm.m[3 * i + 1] * d.y, Rm.m[3 * j + 1], Rm.m[3 * i + 0] * d.x * Rm.m[3 * j + 0]));
  return o;
}
template <class R> static inline V3<R> mat3vec(const M3<R>& A, V3<R> v) {
  return {fma_(A.m[2], v.z, fma_(A.m[1], v.y, A.m[0] * v.x)), fma_(A.m[5], v.z, fma_(A.m[4], v.y, A.m[3] * v.x)),
          fma_(A.m[8], v.z, fma_(A.m[7], v.y, A.m[6] * v.x))};
}

// rigid-body inertia about the common reference point (Iw about com, com offset c, mass m)
template <class R> struct SpatInert { M3<R> Iw; V3<R> c; R m; };

// (reference: src/dynamics.cuh:126-139)
template <class R> static inline void apply_inertia(const SpatInert<R>& I, V3<R> sw, V3<R> sv, V3<R>& fw, V3<R>& fv) {
  R m = I.m; V3<R> c = I.c;
  V3<R> Asw = mat3vec(I.Iw, sw);
  R cc = dot3(c, c);
  R csw = dot3(c, sw);
  Asw = {fma_(m, fma_(-csw, c.x, cc * sw.x), Asw.x), fma_(m, fma_(-csw, c.y, cc * sw.y), Asw.y),
         fma_(m, fma_(-csw, c.z, cc * sw.z), Asw.z)};
  V3<R> mc_sv = cross(c, sv);
  fw = {fma_(m, mc_sv.x, Asw.x), fma_(m, mc_sv.y, Asw.y), fma_(m, mc_sv.z, Asw.z)};
  V3<R> c_sw = cross(c, sw);
  fv = {fma_(m, sv.x, -m * c_sw.x), fma_(m, sv.y, -m * c_sw.y), fma_(m, sv.z, -m * c_sw.z)};
}
// motion x motion (reference: src/dynamics.cuh:142-146)
template <class R> static inline void crossm(V3<R> w1, V3<R> v1, V3<R> w2, V3<R> v2, V3<R>& ow, V3<R>& ov) {
  ow = cross(w1, w2);
  V3<R> a = cross(w1, v2), b = cross(v1, w2);
  ov = {a.x + b.x, a.y + b.y, a.z + b.z};
}
// motion x force (reference: src/dynamics.cuh:148-152)
template <class R> static inline void crossf(V3<R> w1, V3<R> v1, V3<R> n, V3<R> f0, V3<R>& on, V3<R>& of) {
  V3<R> a = cross(w1, n), b = cross(v1, f0);
  on = {a.x + b.x, a.y + b.y, a.z + b.z};
  of = cross(w1, f0);
}

template <class R> static inline Q4<R> ldq(const R* p) { return {p[0], p[1], p[2], p[3]}; }
template <class R> static inline V3<R> ldv(const R* p) { return {p[0], p[1], p[2]}; }

// ---------------------------------------------------------------- forward kinematics
// (reference: src/dynamics.cuh:47-88) The reference composes each body's world frame from its
// parent's, root to leaf: pos = pos_parent + rot(q_parent, body_pos), q = (q_parent (x)
// body_quat) (x) rot(axis, qpos), with the hinge anchor shift pos + rot(q, jnt_pos) -
// rot(q', jnt_pos), the identity since every jnt_pos is 0 (gen_model_tables.py asserts it).
// This restatement composes the same per-body transforms (translation body_pos, rotation
// body_quat (x) rot(axis, qpos); the pelvis: its free-joint pose) by ancestor doubling, the
// association the GPU uses: round r sets T_b <- T_a o T_b with a the 2^r-th ancestor of b, reading
// the transforms of the previous round (tree.h). The per-body transforms are formed in R; the
// compositions of every round but the last run in fp64 for both instantiations, the frames are
// rounded to R once, and the last round (only the arms' distal links have an ancestor left; the
// feet are final before it) and the inertial-frame offsets run in R. In fp32 that keeps the foot
// frames within about one rounding of the exact ones: the foot-ground contact is stiff in the foot
// height, and fp32 compositions (either
// association) move qacc on MuJoCo's contact fixture by up to 2.2e-5 (root -> leaf) or 2.9e-5
// (doubling) relative, fp64 compositions by 1.3e-5 (fp64 everywhere: 9.2e-6). The fp64
// instantiation is pinned against the MuJoCo frames of bench/ref_traj.npz, and
// tests/test_oracle_fixtures.py checks the fp32 frames against the fp32 root -> leaf recursion
// (fk_recursive below).
template <class R> void fk(const R* qpos, R* xpos, R* xquat, R* xipos) {
  using C = typename ComposePrec<R>::type;   // composition precision (fp64)
  V3<C> tp[kNBody];
  Q4<C> tq[kNBody];
  tp[0] = {0, 0, 0};
  tq[0] = {1, 0, 0, 0};
  for (int b = 1; b < kNBody; ++b) {
    const int j = body_jntadr[b], qa = jnt_qposadr[j];
    V3<R> p;
    Q4<R> q;
    if (jnt_type[j] == 0) {
      p = {qpos[qa], qpos[qa + 1], qpos[qa + 2]};
      q = qnorm(Q4<R>{qpos[qa + 3], qpos[qa + 4], qpos[qa + 5], qpos[qa + 6]});
    } else {
      p = ldv(&M<R>::body_pos[3 * b]);
      q = qmul(ldq(&M<R>::body_quat[4 * b]), axisangle(ldv(&M<R>::jnt_axis[3 * j]), qpos[qa]));
    }
    tp[b] = {C(p.x), C(p.y), C(p.z)};
    tq[b] = {C(q.w), C(q.x), C(q.y), C(q.z)};
  }
  // every body composes, with the world body's identity (a = 0) where the 2^r-th ancestor would lie
  // beyond the world: the GPU's branch-free form, equal to leaving the transform unchanged except
  // for the sign of an exact zero
  auto round = [](auto* p, auto* q, int r) {
    using P = typename std::remove_reference<decltype(*p)>::type;
    using Q = typename std::remove_reference<decltype(*q)>::type;
    P op[kNBody];
    Q oq[kNBody];
    std::copy(p, p + kNBody, op);
    std::copy(q, q + kNBody, oq);
    for (int b = 1; b < kNBody; ++b) {
      const int a = kAncestors.a[r][b];
      if (a == 0 && !FkComposeIdentity<R>::value) continue;
      p[b] = vadd(op[a], qrot(oq[a], op[b]));
      q[b] = qmul(oq[a], oq[b]);
    }
  };
  for (int r = 0; r < kFkRounds - 1; ++r) round(tp, tq, r);
  // The last round in R on the frames rounded once (the GPU's form): only the bodies deeper than
  // 2^(kFkRounds-1), the arms' distal links, have an ancestor left, every other body composes with
  // the identity exactly, so the feet keep the fp64 frames rounded once; the inertial-frame offset
  // follows in R from the final frame (the reference's formula on these frames).
  V3<R> fp[kNBody];
  Q4<R> fq[kNBody];
  for (int b = 0; b < kNBody; ++b) {
    fp[b] = {R(tp[b].x), R(tp[b].y), R(tp[b].z)};
    fq[b] = {R(tq[b].w), R(tq[b].x), R(tq[b].y), R(tq[b].z)};
  }
  round(fp, fq, kFkRounds - 1);
  for (int b = 0; b < kNBody; ++b) {
    xpos[3 * b] = fp[b].x; xpos[3 * b + 1] = fp[b].y; xpos[3 * b + 2] = fp[b].z;
    xquat[4 * b] = fq[b].w; xquat[4 * b + 1] = fq[b].x; xquat[4 * b + 2] = fq[b].y; xquat[4 * b + 3] = fq[b].z;
    const V3<R> cw = vadd(fp[b], qrot(fq[b], ldv(&M<R>::body_ipos[3 * b])));
    xipos[3 * b] = cw.x; xipos[3 * b + 1] = cw.y; xipos[3 * b + 2] = cw.z;
  }
  xipos[0] = xipos[1] = xipos[2] = 0;
}

// The reference's root -> leaf recursion, literally (reference: src/dynamics.cuh:47-88): kept to
// check the doubling association against it (tests/test_oracle_fixtures.py).
template <class R> void fk_recursive(const R* qpos, R* xpos, R* xquat, R* xipos) {
  xpos[0] = xpos[1] = xpos[2] = 0;
  xquat[0] = 1; xquat[1] = xquat[2] = xquat[3] = 0;
  for (int b = 1; b < kNBody; ++b) {
    int p = body_parent[b];
    Q4<R> qp = ldq(&xquat[4 * p]);
    V3<R> pp = ldv(&xpos[3 * p]);
    V3<R> pos = vadd(pp, qrot(qp, ldv(&M<R>::body_pos[3 * b])));
    Q4<R> quat = qmul(qp, ldq(&M<R>::body_quat[4 * b]));
    int j = body_jntadr[b];
    int qa = jnt_qposadr[j];
    if (jnt_type[j] == 0) {
      pos = {qpos[qa], qpos[qa + 1], qpos[qa + 2]};
      quat = qnorm(Q4<R>{qpos[qa + 3], qpos[qa + 4], qpos[qa + 5], qpos[qa + 6]});
    } else {
      V3<R> anch = ldv(&M<R>::jnt_pos[3 * j]);
      V3<R> anchor_w = vadd(pos, qrot(quat, anch));
      quat = qmul(quat, axisangle(ldv(&M<R>::jnt_axis[3 * j]), qpos[qa]));
      pos = vsub(anchor_w, qrot(quat, anch));
    }
    xpos[3 * b] = pos.x; xpos[3 * b + 1] = pos.y; xpos[3 * b + 2] = pos.z;
    xquat[4 * b] = quat.w; xquat[4 * b + 1] = quat.x; xquat[4 * b + 2] = quat.y; xquat[4 * b + 3] = quat.z;
    V3<R> cw = vadd(pos, qrot(quat, ldv(&M<R>::body_ipos[3 * b])));
    xipos[3 * b] = cw.x; xipos[3 * b + 1] = cw.y; xipos[3 * b + 2] = cw.z;
  }
  xipos[0] = xipos[1] = xipos[2] = 0;
}

template <class R> struct Frames { R xpos[kNBody * 3], xquat[kNBody * 4], xipos[kNBody * 3]; };

// motion axes about the pelvis origin, world axes (reference: src/aba_bias.cuh:25-43)
template <class R> void motion_axes(const Frames<R>& F, R* S) {
  V3<R> p = ldv(&F.xpos[3]);
  M3<R> R1 = quat2mat(ldq(&F.xquat[4]));
  for (int i = 0; i < kNV * 6; ++i) S[i] = 0;
  for (int j = 0; j < kNJnt; ++j) {
    int b = jnt_bodyid[j], d = jnt_dofadr[j];
    if (jnt_type[j] == 0) {
      S[(d + 0) * 6 + 3] = 1; S[(d + 1) * 6 + 4] = 1; S[(d + 2) * 6 + 5] = 1;
      for (int k = 0; k < 3; ++k) {
        S[(d + 3 + k) * 6 + 0] = R1.m[k]; S[(d + 3 + k) * 6 + 1] = R1.m[3 + k]; S[(d + 3 + k) * 6 + 2] = R1.m[6 + k];
      }
    } else {
      Q4<R> qb = ldq(&F.xquat[4 * b]);
      V3<R> aw = qrot(qb, ldv(&M<R>::jnt_axis[3 * j]));
      V3<R> anchor = vadd(ldv(&F.xpos[3 * b]), qrot(qb, ldv(&M<R>::jnt_pos[3 * j])));
      V3<R> rxa = cross(vsub(anchor, p), aw);
      S[d * 6 + 0] = aw.x; S[d * 6 + 1] = aw.y; S[d * 6 + 2] = aw.z;
      S[d * 6 + 3] = rxa.x; S[d * 6 + 4] = rxa.y; S[d * 6 + 5] = rxa.z;
    }
  }
}

// (reference: src/aba_bias.cuh:45-55)
template <class R> SpatInert<R> body_inertia(const Frames<R>& F, int b) {
  V3<R> p = ldv(&F.xpos[3]);
  SpatInert<R> I;
  M3<R> Ri = quat2mat(qmul(ldq(&F.xquat[4 * b]), ldq(&M<R>::body_iquat[4 * b])));
  I.Iw = world_inertia(Ri, ldv(&M<R>::body_inertia[3 * b]));
  I.c = {F.xipos[3 * b] - p.x, F.xipos[3 * b + 1] - p.y, F.xipos[3 * b + 2] - p.z};
  I.m = M<R>::body_mass[b];
  return I;
}

// ---------------------------------------------------------------- RNE bias (qacc = 0)
// (reference: src/aba_bias.cuh:17-121)
template <class R> void compute_bias(const R* qvel, const Frames<R>& F, R* S, R* bias) {
  motion_axes(F, S);
  SpatInert<R> I[kNBody];
  for (int b = 1; b < kNBody; ++b) I[b] = body_inertia(F, b);
  V3<R> vw[kNBody], vv[kNBody], aw[kNBody], av[kNBody], Sdw[kNV], Sdv[kNV];
  vw[0] = {0, 0, 0}; vv[0] = {0, 0, 0};
  aw[0] = {0, 0, 0}; av[0] = {-M<R>::gravity[0], -M<R>::gravity[1], -M<R>::gravity[2]};
  auto col = [&](int a, V3<R>& sw, V3<R>& sv) {
    sw = {S[a * 6 + 0], S[a * 6 + 1], S[a * 6 + 2]};
    sv = {S[a * 6 + 3], S[a * 6 + 4], S[a * 6 + 5]};
  };
  for (int b = 1; b < kNBody; ++b) {
    int par = body_parent[b];
    V3<R> w = vw[par], v = vv[par];
    int da = body_dofadr[b], dn = body_dofnum[b];
    V3<R> sw, sv;
    if (dn == 6) {
      // translations accumulate normally; all three rotational cdof_dot use the
      // post-translation partial velocity (reference: src/aba_bias.cuh:68-85)
      for (int a = da; a < da + 3; ++a) {
        R qd = qvel[a];
        col(a, sw, sv);
        crossm(w, v, sw, sv, Sdw[a], Sdv[a]);
        w = {fma_(sw.x, qd, w.x), fma_(sw.y, qd, w.y), fma_(sw.z, qd, w.z)};
        v = {fma_(sv.x, qd, v.x), fma_(sv.y, qd, v.y), fma_(sv.z, qd, v.z)};
      }
      V3<R> wr = w, vr = v;
      for (int a = da + 3; a < da + 6; ++a) { col(a, sw, sv); crossm(wr, vr, sw, sv, Sdw[a], Sdv[a]); }
      for (int a = da + 3; a < da + 6; ++a) {
        R qd = qvel[a];
        w = {fma_(S[a * 6 + 0], qd, w.x), fma_(S[a * 6 + 1], qd, w.y), fma_(S[a * 6 + 2], qd, w.z)};
        v = {fma_(S[a * 6 + 3], qd, v.x), fma_(S[a * 6 + 4], qd, v.y), fma_(S[a * 6 + 5], qd, v.z)};
      }
    } else {
      for (int a = da; a < da + dn; ++a) {
        R qd = qvel[a];
        col(a, sw, sv);
        crossm(w, v, sw, sv, Sdw[a], Sdv[a]);
        w = {fma_(sw.x, qd, w.x), fma_(sw.y, qd, w.y), fma_(sw.z, qd, w.z)};
        v = {fma_(sv.x, qd, v.x), fma_(sv.y, qd, v.y), fma_(sv.z, qd, v.z)};
      }
    }
    vw[b] = w; vv[b] = v;
    V3<R> aaw = aw[par], aav = av[par];
    for (int a = da; a < da + dn; ++a) {
      R qd = qvel[a];
      aaw = {fma_(Sdw[a].x, qd, aaw.x), fma_(Sdw[a].y, qd, aaw.y), fma_(Sdw[a].z, qd, aaw.z)};
      aav = {fma_(Sdv[a].x, qd, aav.x), fma_(Sdv[a].y, qd, aav.y), fma_(Sdv[a].z, qd, aav.z)};
    }
    aw[b] = aaw; av[b] = aav;
  }
  V3<R> fw[kNBody], fv[kNBody];
  for (int b = 1; b < kNBody; ++b) {
    V3<R> Iaw, Iav, Ivw, Ivv, cw, cv;
    apply_inertia(I[b], aw[b], av[b], Iaw, Iav);
    apply_inertia(I[b], vw[b], vv[b], Ivw, Ivv);
    crossf(vw[b], vv[b], Ivw, Ivv, cw, cv);
    fw[b] = {Iaw.x + cw.x, Iaw.y + cw.y, Iaw.z + cw.z};
    fv[b] = {Iav.x + cv.x, Iav.y + cv.y, Iav.z + cv.z};
  }
  for (int a = 0; a < kNV; ++a) bias[a] = 0;
  for (int b = kNBody - 1; b >= 1; --b) {
    int da = body_dofadr[b], dn = body_dofnum[b];
    for (int a = da; a < da + dn; ++a)
      bias[a] = fma_(S[a * 6 + 5], fv[b].z, fma_(S[a * 6 + 4], fv[b].y, fma_(S[a * 6 + 3], fv[b].x,
                fma_(S[a * 6 + 2], fw[b].z, fma_(S[a * 6 + 1], fw[b].y, S[a * 6 + 0] * fw[b].x)))));
    int par = body_parent[b];
    if (par >= 1) { fw[par] = vadd(fw[par], fw[b]); fv[par] = vadd(fv[par], fv[b]); }
  }
}

// ---------------------------------------------------------------- summation association
// Three kinds of sum are associated differently by the GPU kernel than by the reference's serial
// loops; the algorithm is the same and the results differ at rounding level. g_ref_order selects
// the association: 0 (default) follows the kernel, so the fp32 oracle reproduces the kernel's
// contact path bit for bit; 1 follows the reference's loops. The three:
//  * the contact basis columns (M + dtB)^-1 e_{c,a}: the kernel solves them in the single
//    right-hand-side form (reference src/aba_factor.cuh:121-165, solveM below), the reference in
//    its K = 1 multi-RHS form (src/aba_solvem_multi.cuh:21-125, solveM_multi1);
//  * the PGS row sums: the kernel scales row i by RN(1/A_ii) once and keeps each row's residual
//    r_i = c_i + sum_{j != i} a_ij f_j up to date by one fused multiply-add per row update (see
//    solve_pgs); the reference accumulates b_i + A_i0 f_0 + ... serially with fused multiply-adds
//    and divides by A_ii (src/contact.cuh:159-171);
//  * the control step's energy and action-change penalty: the kernel sums each actuator's terms
//    over the substeps on its own lane (lane = body = actuator + 2) and the lanes by the butterfly,
//    the reference serially over substeps and actuators (src/g1_env.cu:150-151,186-188).
static int g_ref_order = 0;

// The value every lane of a 32-lane group holds after the kernel's group sum: the xor butterfly
// over strides 16, 8, 4, 2, 1 (lane i adds lane i ^ m; additions commute, so lane 0's sum is
// the pairwise tree below).
template <class R> static inline R butterfly32(const R* v) {
  R t[32];
  for (int i = 0; i < 32; ++i) t[i] = v[i];
  for (int m = 16; m >= 1; m >>= 1)
    for (int i = 0; i < m; ++i) t[i] = t[i] + t[i + m];
  return t[0];
}

// ---------------------------------------------------------------- packed symmetric 6x6 helpers
// (reference: src/aba.cuh:15-27)
static inline int symidx(int i, int j) {
  if (i > j) std::swap(i, j);
  return i * 6 - (i * (i - 1)) / 2 + (j - i);
}
template <class R> static inline R dot6(const R* a, const R* b) {
  R s = 0;
  for (int i = 0; i < 6; ++i) s = fma_(a[i], b[i], s);
  return s;
}
template <class R> static inline void symmv6(const R* P, const R* x, R* o) {
  for (int i = 0; i < 6; ++i) {
    R s = 0;
    for (int j = 0; j < 6; ++j) s = fma_(P[symidx(i, j)], x[j], s);
    o[i] = s;
  }
}

// 6x6 spatial inertia about the pelvis origin, 21-packed (reference: src/aba_factor.cuh:53-74)
template <class R> void spatial_inertia6(const Frames<R>& F, int b, R* X) {
  V3<R> p = ldv(&F.xpos[3]);
  M3<R> Ri = quat2mat(qmul(ldq(&F.xquat[4 * b]), ldq(&M<R>::body_iquat[4 * b])));
  M3<R> Iw = world_inertia(Ri, ldv(&M<R>::body_inertia[3 * b]));
  R m = M<R>::body_mass[b];
  V3<R> c{F.xipos[3 * b] - p.x, F.xipos[3 * b + 1] - p.y, F.xipos[3 * b + 2] - p.z};
  R cc = dot3(c, c);
  R A[9];
  for (int i = 0; i < 9; ++i) A[i] = Iw.m[i];
  A[0] = fma_(m, fma_(-c.x, c.x, cc), A[0]); A[1] = fma_(m, -c.x * c.y, A[1]); A[2] = fma_(m, -c.x * c.z, A[2]);
  A[3] = fma_(m, -c.y * c.x, A[3]); A[4] = fma_(m, fma_(-c.y, c.y, cc), A[4]); A[5] = fma_(m, -c.y * c.z, A[5]);
  A[6] = fma_(m, -c.z * c.x, A[6]); A[7] = fma_(m, -c.z * c.y, A[7]); A[8] = fma_(m, fma_(-c.z, c.z, cc), A[8]);
  R Bx[9] = {0, -c.z, c.y, c.z, 0, -c.x, -c.y, c.x, 0};
  R M6[36];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      M6[6 * i + j] = A[3 * i + j];
      M6[6 * i + (j + 3)] = m * Bx[3 * i + j];
      M6[6 * (i + 3) + j] = -m * Bx[3 * i + j];
      M6[6 * (i + 3) + (j + 3)] = (i == j) ? m : R(0);
    }
  for (int i = 0; i < 6; ++i)
    for (int j = i; j < 6; ++j) X[symidx(i, j)] = M6[i * 6 + j];
}

// ---------------------------------------------------------------- ABA factor (M + dt B)
// (reference: src/aba_factor.cuh:26-31)
template <class R> struct Factor { R U[kNBody * 6]; R invD[kNBody]; R U6[36]; R Dfac6[36]; };

// (reference: src/aba_factor.cuh:44-109)
template <class R> void factorize(const Frames<R>& F, const R* S, const R* Bdiag, Factor<R>& fac) {
  R IA[kNBody * 21];
  for (int b = 1; b < kNBody; ++b) spatial_inertia6(F, b, &IA[b * 21]);
  for (int b = kNBody - 1; b >= 2; --b) {
    int par = body_parent[b], d = body_dofadr[b];
    R U[6];
    symmv6(&IA[b * 21], &S[d * 6], U);
    R D = dot6(&S[d * 6], U) + M<R>::dof_armature[d];
    if (Bdiag) D += Bdiag[d];
    R invD = R(1) / D;
    for (int k = 0; k < 6; ++k) fac.U[b * 6 + k] = U[k];
    fac.invD[b] = invD;
    for (int i = 0; i < 6; ++i)
      for (int j = i; j < 6; ++j) IA[par * 21 + symidx(i, j)] += fma_(-(U[i] * U[j]), invD, IA[b * 21 + symidx(i, j)]);
  }
  int d = body_dofadr[1];
  R Dm[36];
  for (int l = 0; l < 6; ++l) {
    R Ul[6];
    symmv6(&IA[21], &S[(d + l) * 6], Ul);
    for (int i = 0; i < 6; ++i) fac.U6[i * 6 + l] = Ul[i];
  }
  for (int k = 0; k < 6; ++k)
    for (int l = 0; l < 6; ++l) {
      R s = 0;
      for (int i = 0; i < 6; ++i) s = fma_(S[(d + k) * 6 + i], fac.U6[i * 6 + l], s);
      Dm[k * 6 + l] = s + (k == l ? (M<R>::dof_armature[d + k] + (Bdiag ? Bdiag[d + k] : R(0))) : R(0));
    }
  for (int i = 0; i < 6; ++i)
    for (int j = 0; j <= i; ++j) {
      R s = Dm[i * 6 + j];
      for (int kk = 0; kk < j; ++kk) s = fma_(-Dm[i * 6 + kk], Dm[j * 6 + kk], s);
      if (i == j) Dm[i * 6 + i] = sqrt_(s); else Dm[i * 6 + j] = s / Dm[j * 6 + j];
    }
  for (int i = 0; i < 36; ++i) fac.Dfac6[i] = Dm[i];
}

// y = (M + dt B)^-1 x, single right-hand side (reference: src/aba_factor.cuh:121-165)
// The parent's bias force pA starts at its first (highest-index) child's term instead of 0 + that
// term: the two differ only in the sign of an exact zero, which nothing downstream observes.
template <class R> void solveM(const Factor<R>& fac, const R* S, const R* x, R* y) {
  R pA[kNBody * 6], a6[kNBody * 6];
  bool started[kNBody] = {};
  for (int i = 0; i < kNBody * 6; ++i) pA[i] = 0;
  for (int b = kNBody - 1; b >= 2; --b) {
    int par = body_parent[b], d = body_dofadr[b];
    const R* U = &fac.U[b * 6];
    R u = x[d] - dot6(&S[d * 6], &pA[b * 6]);
    R ud = u * fac.invD[b];
    for (int k = 0; k < 6; ++k) {
      const R c = fma_(U[k], ud, pA[b * 6 + k]);
      pA[par * 6 + k] = started[par] ? pA[par * 6 + k] + c : c;
    }
    started[par] = true;
  }
  {
    int d = body_dofadr[1];
    R ap[6] = {0, 0, 0, 0, 0, 0};
    R rhs[6];
    for (int k = 0; k < 6; ++k) {
      R uk = x[d + k] - dot6(&S[(d + k) * 6], &pA[6]);
      R UTa = 0;
      for (int i = 0; i < 6; ++i) UTa = fma_(fac.U6[i * 6 + k], ap[i], UTa);
      rhs[k] = uk - UTa;
    }
    R qdd[6];
    const R* L = fac.Dfac6;
    for (int i = 0; i < 6; ++i) {
      R s = rhs[i];
      for (int k = 0; k < i; ++k) s = fma_(-L[i * 6 + k], qdd[k], s);
      qdd[i] = s / L[i * 6 + i];
    }
    for (int i = 5; i >= 0; --i) {
      R s = qdd[i];
      for (int k = i + 1; k < 6; ++k) s = fma_(-L[k * 6 + i], qdd[k], s);
      qdd[i] = s / L[i * 6 + i];
    }
    for (int k = 0; k < 6; ++k) y[d + k] = qdd[k];
    for (int i = 0; i < 6; ++i) {
      R Sq = 0;
      for (int k = 0; k < 6; ++k) Sq = fma_(S[(d + k) * 6 + i], qdd[k], Sq);
      a6[6 + i] = Sq;   // ap = 0 (no 0 + x)
    }
  }
  for (int b = 2; b < kNBody; ++b) {
    int par = body_parent[b], d = body_dofadr[b];
    R ap[6];
    for (int k = 0; k < 6; ++k) ap[k] = a6[par * 6 + k];
    const R* U = &fac.U[b * 6];
    R u = x[d] - dot6(&S[d * 6], &pA[b * 6]);
    R qdd = (u - dot6(U, ap)) * fac.invD[b];
    y[d] = qdd;
    for (int i = 0; i < 6; ++i) a6[b * 6 + i] = fma_(S[d * 6 + i], qdd, ap[i]);
  }
}

// Same map with the multi-RHS kernel's per-column operation order at K = 1, the form the
// contact basis solves use (reference: src/aba_solvem_multi.cuh:21-125).
template <class R> void solveM_multi1(const Factor<R>& fac, const R* S, const R* x, R* y) {
  R pA[kNBody * 6], a6[kNBody * 6];
  for (int i = 0; i < kNBody * 6; ++i) pA[i] = 0;
  for (int b = kNBody - 1; b >= 2; --b) {
    int par = body_parent[b], d = body_dofadr[b];
    const R* U = &fac.U[b * 6];
    const R* Sd = &S[d * 6];
    R ud = x[d];
    for (int i = 0; i < 6; ++i) ud = fma_(-Sd[i], pA[b * 6 + i], ud);
    ud *= fac.invD[b];
    for (int i = 0; i < 6; ++i) pA[par * 6 + i] += fma_(U[i], ud, pA[b * 6 + i]);
  }
  {
    int d = body_dofadr[1];
    R qdd[6];
    for (int i = 0; i < 6; ++i) {
      R s = 0;
      for (int j = 0; j < 6; ++j) s = fma_(S[(d + i) * 6 + j], pA[6 + j], s);
      qdd[i] = x[d + i] - s;
    }
    const R* L = fac.Dfac6;
    for (int i = 0; i < 6; ++i) {
      R s = qdd[i];
      for (int k = 0; k < i; ++k) s = fma_(-L[i * 6 + k], qdd[k], s);
      qdd[i] = s / L[i * 6 + i];
    }
    for (int i = 5; i >= 0; --i) {
      R s = qdd[i];
      for (int k = i + 1; k < 6; ++k) s = fma_(-L[k * 6 + i], qdd[k], s);
      qdd[i] = s / L[i * 6 + i];
    }
    for (int k = 0; k < 6; ++k) y[d + k] = qdd[k];
    for (int i = 0; i < 6; ++i) {
      R Sq = 0;
      for (int k = 0; k < 6; ++k) Sq = fma_(S[(d + k) * 6 + i], qdd[k], Sq);
      a6[6 + i] = Sq;
    }
  }
  for (int b = 2; b < kNBody; ++b) {
    int par = body_parent[b], d = body_dofadr[b];
    const R* U = &fac.U[b * 6];
    const R* Sd = &S[d * 6];
    R qdd = x[d];
    for (int i = 0; i < 6; ++i) qdd -= fma_(U[i], a6[par * 6 + i], Sd[i] * pA[b * 6 + i]);
    qdd *= fac.invD[b];
    y[d] = qdd;
    for (int i = 0; i < 6; ++i) a6[b * 6 + i] = fma_(Sd[i], qdd, a6[par * 6 + i]);
  }
}

// Dense joint-space inertia (CRBA + armature), a test-only closed-form check of the factor
// (reference: src/dynamics.cuh:199-245).
template <class R> void mass_matrix(const Frames<R>& F, const R* S, R* Mout) {
  R Icp[kNBody][36];
  for (int b = 1; b < kNBody; ++b) {
    R X[21];
    spatial_inertia6(F, b, X);
    for (int i = 0; i < 6; ++i)
      for (int j = 0; j < 6; ++j) Icp[b][6 * i + j] = X[symidx(i, j)];
  }
  for (int b = kNBody - 1; b >= 1; --b) {
    int par = body_parent[b];
    if (par >= 1)
      for (int k = 0; k < 36; ++k) Icp[par][k] += Icp[b][k];
  }
  for (int i = 0; i < kNV * kNV; ++i) Mout[i] = 0;
  for (int b = 1; b < kNBody; ++b) {
    int da = body_dofadr[b], dn = body_dofnum[b];
    for (int a = da; a < da + dn; ++a) {
      R Fv[6];
      for (int i = 0; i < 6; ++i) {
        R s = 0;
        for (int k = 0; k < 6; ++k) s += Icp[b][6 * i + k] * S[a * 6 + k];
        Fv[i] = s;
      }
      for (int j = b; j >= 1; j = body_parent[j]) {
        int dj = body_dofadr[j], djn = body_dofnum[j];
        for (int c2 = dj; c2 < dj + djn; ++c2) {
          R v = 0;
          for (int k = 0; k < 6; ++k) v += S[c2 * 6 + k] * Fv[k];
          Mout[a * kNV + c2] = v;
          Mout[c2 * kNV + a] = v;
        }
      }
    }
  }
  for (int a = 0; a < kNV; ++a) Mout[a * kNV + a] += M<R>::dof_armature[a];
}

// ---------------------------------------------------------------- foot contact
// MuJoCo solimp impedance (reference: src/contact.cuh:97-109)
template <class R> R foot_impedance(R pos) {
  const R* si = M<R>::foot_solimp;
  R dmin = si[0], dmax = si[1], width = si[2], mid = si[3], power = si[4];
  R x = fabs_(pos) / width;
  R y;
  if (x >= R(1)) y = 1;
  else {
    R a = R(1) / pow_(mid, power - R(1));
    R b = R(1) / pow_(R(1) - mid, power - R(1));
    y = (x < mid) ? a * pow_(x, power) : fma_(-b, pow_(R(1) - x, power), R(1));
  }
  return fma_(y, dmax - dmin, dmin);
}

static inline uint64_t bits_of(float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; }
static inline uint64_t bits_of(double x) { uint64_t u; std::memcpy(&u, &x, 8); return u; }

// Sweeps between the fresh residuals of the kernel's PGS association (solve_pgs).
constexpr int kPgsRefresh = 8;

// Projected Gauss-Seidel on min 0.5 f'Af + f'b, f >= 0 (reference: src/contact.cuh:159-171):
// f_i = max(0, -(b_i + sum_{j != i} A_ij f_j) / A_ii), rows in order, `iters` sweeps from f = 0.
// Reference association (g_ref_order, or n > 32): the row sum b_i + A_i0 f_0 + ... serially in
// fused multiply-adds, minus A_ii f_i, divided by A_ii.
// Kernel association (n <= 32): row i is scaled once by y_i = RN(1/A_ii), a_ij = RN(A_ij y_i) off
// the diagonal (a_ii = 0) and c_i = RN(b_i y_i), and each row keeps its residual
// r_i = c_i + sum_j a_ij f_j current: r = c at f = 0; a row update sets f_i = max(0, -r_i) and adds
// a_ji d to every r_j (one fma each, j = 0..31 in the kernel's lanes, d = RN(f_i new - f_i old)).
// So a row costs no sum and no division. Every kPgsRefresh-th sweep starts from fresh residuals
// (r_i = c_i, then fma(a_ik, f_k, r_i) over k in order), which bounds the rounding carried by the
// updates over long solves; and the sweeps stop after the first sweep that changes no f bit for
// bit. Before a fresh residual that stop changes nothing (the next sweep would repeat the last
// exactly); after one it is part of this association. Against the reference association: qacc
// within 5e-6 relative on the gate and config-2 state families at 8 sweeps, and the MuJoCo contact
// fixture at 2000 sweeps as close as with the reference's sums (tests/test_oracle_fixtures.py,
// tests/test_gpu_parity.py).
template <class R> void solve_pgs(const R* A, const R* b, R* f, int n, int iters) {
  for (int i = 0; i < n; ++i) f[i] = 0;
  if (g_ref_order || n > 32) {
    for (int it = 0; it < iters; ++it)
      for (int i = 0; i < n; ++i) {
        R Aii = A[i * n + i];
        R ri = b[i];
        for (int j = 0; j < n; ++j) ri = fma_(A[i * n + j], f[j], ri);
        ri = fma_(-Aii, f[i], ri);
        R fi = -ri / Aii;
        f[i] = fi > R(0) ? fi : R(0);
      }
    return;
  }
  R a[32][32], c[32], r[32];
  for (int i = 0; i < n; ++i) {
    const R y = R(1) / A[i * n + i];
    for (int j = 0; j < n; ++j) a[i][j] = j == i ? R(0) : A[i * n + j] * y;
    c[i] = b[i] * y;
    r[i] = c[i];
  }
  for (int it = 0; it < iters; ++it) {
    if (it > 0 && it % kPgsRefresh == 0)
      for (int i = 0; i < n; ++i) {
        R t = c[i];
        for (int k = 0; k < n; ++k) t = fma_(a[i][k], f[k], t);
        r[i] = t;
      }
    bool moved = false;
    for (int i = 0; i < n; ++i) {
      const R t = -r[i];
      const R fn = t > R(0) ? t : R(0);
      const R d = fn - f[i];
      if (bits_of(fn) != bits_of(f[i])) moved = true;
      f[i] = fn;
      for (int j = 0; j < n; ++j) r[j] = fma_(a[j][i], d, r[j]);
    }
    if (!moved) break;
  }
}

// Intermediates of one contact solve, exposed for debugging and tests.
template <class R> struct ContactDebug {
  int ncon;
  R A[kMaxEfc * kMaxEfc], b[kMaxEfc], f[kMaxEfc], R_[kMaxEfc], aref[kMaxEfc];
  R qacc_smooth[kNV];
};

// Full per-substep generalized acceleration: (M + dtB)^-1(-bias + tau) plus the foot-ground
// pyramidal contact correction (reference: src/env_qacc.cuh:27-212). `mu` is the friction
// coefficient (model value 0.6; configurable for the contact-only benchmark configuration).
template <class R>
int env_qacc(const R* qp, const R* qv, const Frames<R>& F, const R* tau, const R* Bdt, R* S, R* qacc, int pgs,
             R mu, ContactDebug<R>* dbg = nullptr, bool contact = true) {
  (void)qp;
  R bias[kNV], negbias[kNV], qacc_s[kNV];
  compute_bias(qv, F, S, bias);
  for (int i = 0; i < kNV; ++i) negbias[i] = -bias[i];
  Factor<R> fac;
  factorize(F, S, Bdt, fac);
  R rhs[kNV];
  for (int i = 0; i < kNV; ++i) rhs[i] = negbias[i] + tau[i];
  solveM(fac, S, rhs, qacc_s);
  if (dbg) { std::memcpy(dbg->qacc_smooth, qacc_s, sizeof(qacc_s)); dbg->ncon = 0; }
  if (!contact) {   // smooth-only evaluation (no foot contacts)
    for (int i = 0; i < kNV; ++i) qacc[i] = qacc_s[i];
    return 0;
  }

  // detect: 8 foot spheres vs the z = 0 plane (reference: src/contact.cuh:31-46)
  int cbody[kNFoot]; R cpt[kNFoot][3], cpen[kNFoot], invw0[kNFoot];
  int ncon = 0;
  for (int s = 0; s < kNFoot; ++s) {
    int b = foot_body[s];
    V3<R> c = vadd(ldv(&F.xpos[3 * b]), qrot(ldq(&F.xquat[4 * b]), ldv(&M<R>::foot_lpos[3 * s])));
    R pen = c.z - M<R>::foot_radius;
    if (pen < R(0)) {
      cbody[ncon] = b; cpen[ncon] = pen;
      cpt[ncon][0] = c.x; cpt[ncon][1] = c.y; cpt[ncon][2] = pen * R(0.5);
      invw0[ncon] = M<R>::foot_invweight0[s];   // (reference: src/env_qacc.cuh:59-65)
      ++ncon;
    }
  }
  if (ncon == 0) {
    for (int i = 0; i < kNV; ++i) qacc[i] = qacc_s[i];
    return 0;
  }
  V3<R> p = ldv(&F.xpos[3]);
  const int nefc = 4 * ncon;
  const R* solref = M<R>::foot_solref;
  const R dmaxRA = M<R>::foot_solimp[1];
  const R bcoef = R(2) / (dmaxRA * solref[0]);
  const R kcoef = R(1) / (dmaxRA * dmaxRA * solref[0] * solref[0] * solref[1] * solref[1]);
  const R pyrRA = (R(1) + mu * mu) * (R(2) * mu * mu / M<R>::foot_impratio);

  // ancestor dof list of each contact body, walked foot -> root (reference: src/env_qacc.cuh:83-96)
  constexpr int CDS = kContactDofs;
  int cdof[kNFoot][CDS], cnd[kNFoot];
  for (int c = 0; c < ncon; ++c) {
    int n = 0;
    for (int b = cbody[c]; b >= 1; b = body_parent[b])
      for (int a = body_dofadr[b]; a < body_dofadr[b] + body_dofnum[b]; ++a) cdof[c][n++] = a;
    cnd[c] = n;
  }
  // PASS 1: 3-basis rows e0 = jc.z, e1 = mu jc.y, e2 = -mu jc.x, bb = e.qacc_s, aref, R
  // (reference: src/env_qacc.cuh:107-136; point Jacobian: src/contact.cuh:51-57)
  R Eb[kNFoot][3][CDS], bb[kNFoot][3], Rr[kMaxEfc], aref[kMaxEfc];
  for (int c = 0; c < ncon; ++c) {
    V3<R> pt{cpt[c][0], cpt[c][1], cpt[c][2]};
    V3<R> r = vsub(pt, p);
    R b0 = 0, b1 = 0, b2 = 0, v0 = 0, v1 = 0, v2 = 0;
    for (int k = 0; k < cnd[c]; ++k) {
      int a = cdof[c][k];
      V3<R> w{S[a * 6 + 0], S[a * 6 + 1], S[a * 6 + 2]}, lv{S[a * 6 + 3], S[a * 6 + 4], S[a * 6 + 5]};
      V3<R> jc = vadd(cross(w, r), lv);
      R e0 = jc.z, e1 = mu * jc.y, e2 = -mu * jc.x;
      Eb[c][0][k] = e0; Eb[c][1][k] = e1; Eb[c][2][k] = e2;
      R qa = qacc_s[a];
      b0 = fma_(e0, qa, b0); b1 = fma_(e1, qa, b1); b2 = fma_(e2, qa, b2);
      R qd = qv[a];
      v0 = fma_(e0, qd, v0); v1 = fma_(e1, qd, v1); v2 = fma_(e2, qd, v2);
    }
    bb[c][0] = b0; bb[c][1] = b1; bb[c][2] = b2;
    R pen = cpen[c], imp = foot_impedance(pen);
    R Rc = invw0[c] * pyrRA * (R(1) - imp) / imp;
    R kip = kcoef * imp * pen;
    for (int k = 0; k < 4; ++k) {
      int idx = 4 * c + k;
      Rr[idx] = Rc;
      R dkv = (k == 0) ? v0 + v1 : (k == 1) ? v0 - v1 : (k == 2) ? v0 + v2 : v0 - v2;
      aref[idx] = -bcoef * dkv - kip;
    }
  }
  // PASS 2: m_{c,a} = (M + dtB)^-1 e_{c,a} (reference: src/env_qacc.cuh:143-152; solve form as
  // selected by g_ref_order)
  R Mm[kNFoot][3][kNV];
  for (int c = 0; c < ncon; ++c)
    for (int a = 0; a < 3; ++a) {
      R basis[kNV];
      for (int i = 0; i < kNV; ++i) basis[i] = 0;
      for (int k = 0; k < cnd[c]; ++k) basis[cdof[c][k]] = Eb[c][a][k];
      if (g_ref_order) solveM_multi1(fac, S, basis, Mm[c][a]);
      else solveM(fac, S, basis, Mm[c][a]);
    }
  // A = J M^-1 J' + diag(R) from 3x3 Gram blocks expanded to the 4x4 pyramid blocks,
  // upper blocks copied symmetric (reference: src/env_qacc.cuh:154-192)
  static const R DC[4][3] = {{1, 1, 0}, {1, -1, 0}, {1, 0, 1}, {1, 0, -1}};
  R A[kMaxEfc * kMaxEfc], bvec[kMaxEfc];
  for (int c = 0; c < ncon; ++c) {
    for (int cp = c; cp < ncon; ++cp) {
      R G[3][3];
      for (int a = 0; a < 3; ++a) {
        R g0 = 0, g1 = 0, g2 = 0;
        for (int k = 0; k < cnd[c]; ++k) {
          R v = Eb[c][a][k];
          int dd = cdof[c][k];
          g0 = fma_(v, Mm[cp][0][dd], g0); g1 = fma_(v, Mm[cp][1][dd], g1); g2 = fma_(v, Mm[cp][2][dd], g2);
        }
        G[a][0] = g0; G[a][1] = g1; G[a][2] = g2;
      }
      for (int k = 0; k < 4; ++k) {
        const R* dk = DC[k];
        R t0 = fma_(dk[2], G[2][0], fma_(dk[1], G[1][0], dk[0] * G[0][0]));
        R t1 = fma_(dk[2], G[2][1], fma_(dk[1], G[1][1], dk[0] * G[0][1]));
        R t2 = fma_(dk[2], G[2][2], fma_(dk[1], G[1][2], dk[0] * G[0][2]));
        int i = 4 * c + k;
        for (int kp = 0; kp < 4; ++kp) {
          const R* dq4 = DC[kp];
          R aij = fma_(t2, dq4[2], fma_(t1, dq4[1], t0 * dq4[0]));
          int j = 4 * cp + kp;
          if (i == j) aij += Rr[i];
          A[i * nefc + j] = aij;
          A[j * nefc + i] = aij;
        }
      }
    }
    for (int k = 0; k < 4; ++k) {
      const R* dk = DC[k];
      int i = 4 * c + k;
      bvec[i] = fma_(dk[2], bb[c][2], fma_(dk[1], bb[c][1], dk[0] * bb[c][0])) - aref[i];
    }
  }
  R f[kMaxEfc];
  solve_pgs(A, bvec, f, nefc, pgs);
  // dq = sum_c sum_a fb_c[a] m_{c,a} (reference: src/env_qacc.cuh:199-211)
  R dq[kNV];
  for (int a = 0; a < kNV; ++a) dq[a] = 0;
  for (int c = 0; c < ncon; ++c) {
    R f0 = f[4 * c], f1 = f[4 * c + 1], f2 = f[4 * c + 2], f3 = f[4 * c + 3];
    R fb0 = f0 + f1 + f2 + f3, fb1 = f0 - f1, fb2 = f2 - f3;
    for (int a = 0; a < kNV; ++a) dq[a] += fma_(fb2, Mm[c][2][a], fma_(fb1, Mm[c][1][a], fb0 * Mm[c][0][a]));
  }
  for (int i = 0; i < kNV; ++i) qacc[i] = qacc_s[i] + dq[i];
  if (dbg) {
    dbg->ncon = ncon;
    for (int i = 0; i < nefc * nefc; ++i) dbg->A[i] = A[i];
    for (int i = 0; i < nefc; ++i) { dbg->b[i] = bvec[i]; dbg->f[i] = f[i]; dbg->R_[i] = Rr[i]; dbg->aref[i] = aref[i]; }
  }
  return ncon;
}

// ---------------------------------------------------------------- integration
// q <- normalize(q (x) exp(w dt)), w body-local (reference: src/dynamics.cuh:333-342)
template <class R> void quat_integrate(R* q, V3<R> w, R dt) {
  V3<R> v{w.x * dt, w.y * dt, w.z * dt};
  R ang = sqrt_(fma_(v.z, v.z, fma_(v.y, v.y, v.x * v.x)));
  Q4<R> dq;
  if (ang < R(1e-9)) dq = {R(1), R(0.5) * v.x, R(0.5) * v.y, R(0.5) * v.z};
  else {
    R s = sin_(R(0.5) * ang) / ang;
    dq = {cos_(R(0.5) * ang), v.x * s, v.y * s, v.z * s};
  }
  Q4<R> qn = qnorm(qmul(Q4<R>{q[0], q[1], q[2], q[3]}, dq));
  q[0] = qn.w; q[1] = qn.x; q[2] = qn.y; q[3] = qn.z;
}
// semi-implicit Euler position update (reference: src/dynamics.cuh:345-355)
template <class R> void integrate_pos(R* qpos, const R* qvel, R dt) {
  for (int j = 0; j < kNJnt; ++j) {
    int qa = jnt_qposadr[j], da = jnt_dofadr[j];
    if (jnt_type[j] == 0) {
      qpos[qa] = fma_(dt, qvel[da], qpos[qa]); qpos[qa + 1] = fma_(dt, qvel[da + 1], qpos[qa + 1]);
      qpos[qa + 2] = fma_(dt, qvel[da + 2], qpos[qa + 2]);
      quat_integrate(&qpos[qa + 3], V3<R>{qvel[da + 3], qvel[da + 4], qvel[da + 5]}, dt);
    } else {
      qpos[qa] = fma_(dt, qvel[da], qpos[qa]);
    }
  }
}

// ---------------------------------------------------------------- environment
constexpr int kObs = 100, kAct = 29;

// (reference: src/g1_env.cu:69-81)
template <class R> void compute_obs(const R* qp, const R* qv, const R* pa, R* obs) {
  for (int i = 0; i < 3; ++i) obs[i] = qv[i];
  for (int i = 0; i < 3; ++i) obs[3 + i] = qv[3 + i];
  M3<R> Rb = quat2mat(Q4<R>{qp[3], qp[4], qp[5], qp[6]});
  obs[6] = -Rb.m[6]; obs[7] = -Rb.m[7]; obs[8] = -Rb.m[8];
  for (int i = 0; i < kAct; ++i) obs[9 + i] = qp[act_qadr[i]];
  for (int i = 0; i < kAct; ++i) obs[38 + i] = qv[act_dof[i]];
  for (int i = 0; i < kAct; ++i) obs[67 + i] = pa[i];
  obs[96] = R(0.8); obs[97] = 0; obs[98] = 0; obs[99] = 0;
}

// One control step: S substeps of FK -> PD torque -> env_qacc -> Euler, then reward,
// termination and auto-reset (reference: src/g1_env.cu:118-212). `reset_noise` (29 values in
// [-1,1]) stands in for the reference's per-world curand stream on an auto-reset.
template <class R>
void env_advance(R* lp, R* lv, R* pa, int* pstep, const R* a, const R* reset_noise, int S, int pgs, R mu, R* r_out,
                 int* done_out, int* ncon_hist = nullptr) {
  R target[kAct];
  const R ACT_SCALE = R(0.5);
  for (int i = 0; i < kAct; ++i) {
    R t = fma_(ACT_SCALE, a[i], M<R>::qpos_stand[act_qadr[i]]);
    if (t < M<R>::act_ctrl_lo[i]) t = M<R>::act_ctrl_lo[i];
    if (t > M<R>::act_ctrl_hi[i]) t = M<R>::act_ctrl_hi[i];
    target[i] = t;
  }
  Frames<R> F;
  R Sm[kNV * 6], qacc[kNV], tau[kNV];
  const R dt = M<R>::dt;
  R Bdt[kNV];
  for (int i = 0; i < kNV; ++i) Bdt[i] = 0;
  for (int i = 0; i < kAct; ++i) Bdt[act_dof[i]] = dt * M<R>::act_kd[i];
  R vx_sum = 0, energy = 0;
  R e_act[kAct];   // per-actuator energy over the substeps (kernel association)
  for (int i = 0; i < kAct; ++i) e_act[i] = 0;
  int alive = 1;
  for (int s = 0; s < S; ++s) {
    fk(lp, F.xpos, F.xquat, F.xipos);
    for (int i = 0; i < kNV; ++i) tau[i] = 0;
    for (int i = 0; i < kAct; ++i) {
      int d = act_dof[i];
      R pdt = fma_(-M<R>::act_kd[i], lv[d], M<R>::act_kp[i] * (target[i] - lp[act_qadr[i]]));
      if (pdt < M<R>::act_frc_lo[i]) pdt = M<R>::act_frc_lo[i];
      else if (pdt > M<R>::act_frc_hi[i]) pdt = M<R>::act_frc_hi[i];
      tau[d] = pdt;
      if (g_ref_order) energy += fabs_(pdt * lv[d]);
      else e_act[i] += fabs_(pdt * lv[d]);
    }
    int nc = env_qacc(lp, lv, F, tau, Bdt, Sm, qacc, pgs, mu);
    if (ncon_hist) ncon_hist[nc] += 1;
    for (int i = 0; i < kNV; ++i) {
      R v = fma_(dt, qacc[i], lv[i]);
      if (!isfinite_(v)) v = 0;
      if (v > R(50)) v = R(50); else if (v < R(-50)) v = R(-50);
      lv[i] = v;
    }
    integrate_pos(lp, lv, dt);
    vx_sum += lv[0];
  }
  R vx = vx_sum / R(S);
  R height = lp[2];
  M3<R> Rb = quat2mat(Q4<R>{lp[3], lp[4], lp[5], lp[6]});
  R up = Rb.m[8];
  if (height < R(0.45) || up < R(0.5)) alive = 0;
  R upc = up < R(0) ? R(0) : (up > R(1) ? R(1) : up);
  R vx_c = vx > R(0.8) ? R(0.8) : vx;
  if (vx_c < R(0)) vx_c = 0;
  R r_vel = R(1) * vx_c * upc;
  R r_lat = -R(0.2) * fabs_(lv[1]) - R(0.05) * fabs_(lv[5]);
  R r_up = R(0.3) * upc;
  R r_h = -R(0.5) * fabs_(height - R(0.78));
  R act_pen = 0;
  if (g_ref_order) {
    for (int i = 0; i < kAct; ++i) { R da = a[i] - pa[i]; act_pen += da * da; }
  } else {
    // actuator i on lane i + 2 (lanes 0, 1 and 31 carry no actuator)
    R le[32], lp[32];
    for (int k = 0; k < 32; ++k) le[k] = lp[k] = R(0);
    for (int i = 0; i < kAct; ++i) {
      R da = a[i] - pa[i];
      le[i + 2] = e_act[i];
      lp[i + 2] = da * da;
    }
    energy = butterfly32(le);
    act_pen = butterfly32(lp);
  }
  if (act_pen > R(10)) act_pen = R(10);
  R r;
  if (alive) r = R(1) + r_vel + r_lat + r_up + r_h - R(0.005) * act_pen - R(1e-4) * energy;
  else r = R(-5);
  *pstep += 1;
  int won = (alive && lp[0] >= R(5));
  if (won) r += R(50);
  int d_flag = (!alive || won || *pstep >= 1000) ? 1 : 0;
  for (int i = 0; i < kAct; ++i) pa[i] = a[i];
  if (d_flag) {
    for (int i = 0; i < kNQ; ++i) lp[i] = M<R>::qpos_stand[i];
    for (int i = 0; i < kAct; ++i) lp[act_qadr[i]] += R(0.05) * reset_noise[i];
    for (int i = 0; i < kNV; ++i) lv[i] = 0;
    for (int i = 0; i < kAct; ++i) pa[i] = 0;
    *pstep = 0;
  }
  *r_out = r;
  *done_out = d_flag;
}

// ---------------------------------------------------------------- policy MLP
// Layer spec: nl hidden layers with widths hid[0..nl-1], activation act (0 = tanh, 1 = ELU),
// heads mu (ACT) and value (1) off the last hidden layer, then log_std[ACT]. Packed in torch
// parameter order W0,b0,...,Wmu,bmu,Wv,bv,log_std, nn.Linear weights [out,in] row-major
// (reference: src/g1_env.cu:219-239; packing scripts/ppo_fused.py:35-44).
struct PolicySpec { int nl; int hid[4]; int act; };

inline long policy_params(const PolicySpec& ps) {
  long n = 0; int in = kObs;
  for (int l = 0; l < ps.nl; ++l) { n += (long)ps.hid[l] * in + ps.hid[l]; in = ps.hid[l]; }
  return n + (long)kAct * in + kAct + in + 1 + kAct;
}

template <class R> void mlp_forward(const R* W, const PolicySpec& ps, const R* x, R* mu, R* ls, R* val) {
  std::vector<R> cur(x, x + kObs), nxt;
  const R* p = W;
  int in = kObs;
  for (int l = 0; l < ps.nl; ++l) {
    int out = ps.hid[l];
    const R* Wl = p; const R* bl = Wl + (long)out * in;
    nxt.assign(out, R(0));
    for (int o = 0; o < out; ++o) {
      R s = bl[o];
      const R* row = Wl + (long)o * in;
      for (int i = 0; i < in; ++i) s += row[i] * cur[i];
      nxt[o] = ps.act == 0 ? tanh_(s) : (s > R(0) ? s : expm1_(s));
    }
    p = bl + out; in = out; cur.swap(nxt);
  }
  const R* Wmu = p; const R* bmu = Wmu + (long)kAct * in;
  const R* Wv = bmu + kAct; const R* bv = Wv + in; const R* lsp = bv + 1;
  for (int o = 0; o < kAct; ++o) {
    R s = bmu[o];
    const R* row = Wmu + (long)o * in;
    for (int i = 0; i < in; ++i) s += row[i] * cur[i];
    mu[o] = s;
  }
  R sv = bv[0];
  for (int i = 0; i < in; ++i) sv += Wv[i] * cur[i];
  *val = sv;
  for (int o = 0; o < kAct; ++o) ls[o] = lsp[o];
}

// obs normalisation with frozen stats, clamp +-10 (reference: src/g1_env.cu:298-302)
template <class R> void normalize_obs(const R* o, const R* mean, const R* var, R* no) {
  for (int i = 0; i < kObs; ++i) {
    R z = (o[i] - mean[i]) / sqrt_(var[i] + R(1e-8));
    if (z < R(-10)) z = R(-10); else if (z > R(10)) z = R(10);
    no[i] = z;
  }
}

// One world's fused rollout with pre-generated noise (reference: src/g1_env.cu:278-338).
// act_noise/reset_noise are [H][N][29]; trajectory outputs are [H][N][...].
template <class R>
void rollout_world(int w, int N, int H, int S, int pgs, R mu_fric, R* qp, R* qv, R* pa, int* steps, const R* W,
                   const PolicySpec& ps, const R* mean, const R* var, const R* act_noise, const R* reset_noise, R* O,
                   R* A, R* LP, R* V, R* Rw, R* D, R* Vlast, int* ncon_hist) {
  R* lp = qp + (long)w * kNQ; R* lv = qv + (long)w * kNV; R* lpa = pa + (long)w * kAct;
  int step = steps[w];
  const R LOG2PI = R(1.8378770664093453);
  R o[kObs], no[kObs], mu[kAct], ls[kAct], val, a[kAct];
  for (int t = 0; t < H; ++t) {
    compute_obs(lp, lv, lpa, o);
    normalize_obs(o, mean, var, no);
    long ob = ((long)t * N + w);
    for (int i = 0; i < kObs; ++i) O[ob * kObs + i] = o[i];
    mlp_forward(W, ps, no, mu, ls, &val);
    R lpsum = 0;
    const R* nz = act_noise + ob * kAct;
    for (int i = 0; i < kAct; ++i) {
      R sd = exp_(ls[i]);
      a[i] = mu[i] + sd * nz[i];
      lpsum += -R(0.5) * nz[i] * nz[i] - ls[i] - R(0.5) * LOG2PI;
    }
    for (int i = 0; i < kAct; ++i) A[ob * kAct + i] = a[i];
    LP[ob] = lpsum; V[ob] = val;
    R r; int dfl;
    env_advance(lp, lv, lpa, &step, a, reset_noise + ob * kAct, S, pgs, mu_fric, &r, &dfl, ncon_hist);
    Rw[ob] = r; D[ob] = R(dfl);
  }
  compute_obs(lp, lv, lpa, o);
  normalize_obs(o, mean, var, no);
  mlp_forward(W, ps, no, mu, ls, &val);
  Vlast[w] = val;
  steps[w] = step;
}

}  // namespace orc

// ====================================================================== C ABI (ctypes)
using namespace orc;

template <class R> static void fk_batch(int n, const R* qpos, R* xpos, R* xquat, R* xipos) {
  for (int w = 0; w < n; ++w)
    fk(qpos + (long)w * kNQ, xpos + (long)w * kNBody * 3, xquat + (long)w * kNBody * 4, xipos + (long)w * kNBody * 3);
}
template <class R> static void bias_batch(int n, const R* qpos, const R* qvel, R* S, R* bias) {
  for (int w = 0; w < n; ++w) {
    Frames<R> F;
    fk(qpos + (long)w * kNQ, F.xpos, F.xquat, F.xipos);
    compute_bias(qvel + (long)w * kNV, F, S + (long)w * kNV * 6, bias + (long)w * kNV);
  }
}
template <class R> static void mass_batch(int n, const R* qpos, R* Mo) {
  for (int w = 0; w < n; ++w) {
    Frames<R> F; R S[kNV * 6];
    fk(qpos + (long)w * kNQ, F.xpos, F.xquat, F.xipos);
    motion_axes(F, S);
    mass_matrix(F, S, Mo + (long)w * kNV * kNV);
  }
}
template <class R> static void solve_batch(int n, const R* qpos, const R* Bdt, const R* x, R* y, int multi) {
  for (int w = 0; w < n; ++w) {
    Frames<R> F; R S[kNV * 6]; Factor<R> fac;
    fk(qpos + (long)w * kNQ, F.xpos, F.xquat, F.xipos);
    motion_axes(F, S);
    factorize(F, S, Bdt, fac);
    if (multi) solveM_multi1(fac, S, x + (long)w * kNV, y + (long)w * kNV);
    else solveM(fac, S, x + (long)w * kNV, y + (long)w * kNV);
  }
}
template <class R>
static void qacc_batch(int n, const R* qpos, const R* qvel, const R* tau, const R* Bdt, int pgs, R mu, R* qacc,
                       int* ncon, int nthreads, int contact) {
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 16)
  for (int w = 0; w < n; ++w) {
    Frames<R> F; R S[kNV * 6];
    fk(qpos + (long)w * kNQ, F.xpos, F.xquat, F.xipos);
    int nc = env_qacc(qpos + (long)w * kNQ, qvel + (long)w * kNV, F, tau + (long)w * kNV, Bdt, S, qacc + (long)w * kNV,
                      pgs, mu, (ContactDebug<R>*)nullptr, contact != 0);
    if (ncon) ncon[w] = nc;
  }
}
// nsub substeps for a batch driven by a generalized force tau on the hinge dofs (FK -> env_qacc ->
// v += dt qacc, optionally with the env's NaN/clamp guard -> integrate), damped or plain factor,
// contact on or off: the
// counterpart of the library's dynamics benchmark (smooth dynamics: reference src/sim_aba.cu:19-38).
template <class R>
static void dyn_batch(int n, R* qpos, R* qvel, const R* tau, int nsub, int contact, int damped, int guard, int pgs,
                      R mu, R* qacc_out, int* ncon, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 16)
  for (int w = 0; w < n; ++w) {
    R* lp = qpos + (long)w * kNQ; R* lv = qvel + (long)w * kNV;
    const R* tw = tau + (long)w * kNV;
    Frames<R> F; R S[kNV * 6], t[kNV], qacc[kNV], Bdt[kNV];
    const R dt = M<R>::dt;
    for (int i = 0; i < kNV; ++i) { Bdt[i] = 0; t[i] = i < 6 ? R(0) : tw[i]; }
    for (int i = 0; i < kAct; ++i) Bdt[act_dof[i]] = dt * M<R>::act_kd[i];
    int nc = 0;
    for (int s = 0; s < nsub; ++s) {
      fk(lp, F.xpos, F.xquat, F.xipos);
      nc = env_qacc(lp, lv, F, t, damped ? Bdt : nullptr, S, qacc, pgs, mu, (ContactDebug<R>*)nullptr, contact != 0);
      for (int i = 0; i < kNV; ++i) {
        R v = fma_(dt, qacc[i], lv[i]);
        if (guard) {   // (reference: src/g1_env.cu:154-160)
          if (!isfinite_(v)) v = 0;
          if (v > R(50)) v = R(50); else if (v < R(-50)) v = R(-50);
        }
        lv[i] = v;
      }
      integrate_pos(lp, lv, dt);
    }
    if (ncon) ncon[w] = nc;
    if (qacc_out) for (int i = 0; i < kNV; ++i) qacc_out[(long)w * kNV + i] = qacc[i];
  }
}

// One substep for a batch (FK -> PD torque with clamp -> env_qacc -> Euler with NaN/clamp ->
// integrate), the teacher-forced unit of the per-substep parity gate (reference:
// src/g1_env.cu:141-163). target[n][29] are PD joint targets.
template <class R>
static void substep_batch(int n, R* qpos, R* qvel, const R* target, int pgs, R mu, R* qacc_out, int* ncon,
                          int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 16)
  for (int w = 0; w < n; ++w) {
    R* lp = qpos + (long)w * kNQ; R* lv = qvel + (long)w * kNV;
    const R* tg = target + (long)w * kAct;
    Frames<R> F; R S[kNV * 6], tau[kNV], qacc[kNV], Bdt[kNV];
    const R dt = M<R>::dt;
    for (int i = 0; i < kNV; ++i) Bdt[i] = 0;
    for (int i = 0; i < kAct; ++i) Bdt[act_dof[i]] = dt * M<R>::act_kd[i];
    fk(lp, F.xpos, F.xquat, F.xipos);
    for (int i = 0; i < kNV; ++i) tau[i] = 0;
    for (int i = 0; i < kAct; ++i) {
      int d = act_dof[i];
      R pdt = fma_(-M<R>::act_kd[i], lv[d], M<R>::act_kp[i] * (tg[i] - lp[act_qadr[i]]));
      if (pdt < M<R>::act_frc_lo[i]) pdt = M<R>::act_frc_lo[i];
      else if (pdt > M<R>::act_frc_hi[i]) pdt = M<R>::act_frc_hi[i];
      tau[d] = pdt;
    }
    int nc = env_qacc(lp, lv, F, tau, Bdt, S, qacc, pgs, mu);
    if (ncon) ncon[w] = nc;
    for (int i = 0; i < kNV; ++i) {
      R v = fma_(dt, qacc[i], lv[i]);
      if (!isfinite_(v)) v = 0;
      if (v > R(50)) v = R(50); else if (v < R(-50)) v = R(-50);
      lv[i] = v;
    }
    integrate_pos(lp, lv, dt);
    if (qacc_out) for (int i = 0; i < kNV; ++i) qacc_out[(long)w * kNV + i] = qacc[i];
  }
}

// Smooth-dynamics trajectory: qacc = M^-1(-bias), semi-implicit Euler, no actuation or contact
// (the reference's M0/ABA harness: src/dynamics.cu:8-60, src/sim_aba.cu:19-60).
template <class R> static void smooth_traj(const R* q0, const R* v0, int nsteps, R* qout, R* vout) {
  R lp[kNQ], lv[kNV], S[kNV * 6], bias[kNV], rhs[kNV], qacc[kNV];
  std::memcpy(lp, q0, sizeof(lp)); std::memcpy(lv, v0, sizeof(lv));
  std::memcpy(qout, lp, sizeof(lp)); if (vout) std::memcpy(vout, lv, sizeof(lv));
  for (int t = 0; t < nsteps; ++t) {
    Frames<R> F; Factor<R> fac;
    fk(lp, F.xpos, F.xquat, F.xipos);
    compute_bias(lv, F, S, bias);
    factorize(F, S, (const R*)nullptr, fac);
    for (int i = 0; i < kNV; ++i) rhs[i] = -bias[i];
    solveM(fac, S, rhs, qacc);
    for (int i = 0; i < kNV; ++i) lv[i] = fma_(M<R>::dt, qacc[i], lv[i]);
    integrate_pos(lp, lv, M<R>::dt);
    std::memcpy(qout + (long)(t + 1) * kNQ, lp, sizeof(lp));
    if (vout) std::memcpy(vout + (long)(t + 1) * kNV, lv, sizeof(lv));
  }
}

// Implicit-PD trajectory with per-step joint targets, contacts ignored (the reference's
// implicitfast gate: src/test_implicit.cu:42-69). Bdt = dt * Bdiag.
template <class R> static void implicit_traj(const R* q0, const R* v0, const R* Bdt, const R* targets, int nsteps,
                                             R* qout, R* vout) {
  R lp[kNQ], lv[kNV], S[kNV * 6], bias[kNV], rhs[kNV], qacc[kNV], tau[kNV];
  std::memcpy(lp, q0, sizeof(lp)); std::memcpy(lv, v0, sizeof(lv));
  std::memcpy(qout, lp, sizeof(lp)); std::memcpy(vout, lv, sizeof(lv));
  for (int t = 0; t < nsteps; ++t) {
    const R* tg = targets + (long)t * kAct;
    Frames<R> F; Factor<R> fac;
    fk(lp, F.xpos, F.xquat, F.xipos);
    for (int i = 0; i < kNV; ++i) tau[i] = 0;
    for (int i = 0; i < kAct; ++i) {
      int d = act_dof[i];
      R pdt = fma_(-M<R>::act_kd[i], lv[d], M<R>::act_kp[i] * (tg[i] - lp[act_qadr[i]]));
      if (pdt < M<R>::act_frc_lo[i]) pdt = M<R>::act_frc_lo[i];
      else if (pdt > M<R>::act_frc_hi[i]) pdt = M<R>::act_frc_hi[i];
      tau[d] = pdt;
    }
    compute_bias(lv, F, S, bias);
    factorize(F, S, Bdt, fac);
    for (int i = 0; i < kNV; ++i) rhs[i] = -bias[i] + tau[i];
    solveM(fac, S, rhs, qacc);
    for (int i = 0; i < kNV; ++i) lv[i] = fma_(M<R>::dt, qacc[i], lv[i]);
    integrate_pos(lp, lv, M<R>::dt);
    std::memcpy(qout + (long)(t + 1) * kNQ, lp, sizeof(lp));
    std::memcpy(vout + (long)(t + 1) * kNV, lv, sizeof(lv));
  }
}

extern "C" {

void orc_set_reference_order(int on) { g_ref_order = on ? 1 : 0; }

void orc_smooth_traj_f(const float* q0, const float* v0, int n, float* qo, float* vo) { smooth_traj(q0, v0, n, qo, vo); }
void orc_smooth_traj_d(const double* q0, const double* v0, int n, double* qo, double* vo) { smooth_traj(q0, v0, n, qo, vo); }
void orc_implicit_traj_f(const float* q0, const float* v0, const float* Bdt, const float* tg, int n, float* qo,
                         float* vo) { implicit_traj(q0, v0, Bdt, tg, n, qo, vo); }
void orc_implicit_traj_d(const double* q0, const double* v0, const double* Bdt, const double* tg, int n, double* qo,
                         double* vo) { implicit_traj(q0, v0, Bdt, tg, n, qo, vo); }

// the oracle's sine and cosine of floats (fp64 libm, rounded once)
void orc_sincos_f(long n, const float* x, float* sn, float* cs) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) { sn[i] = sin_(x[i]); cs[i] = cos_(x[i]); }
}

int orc_nbody() { return kNBody; }
int orc_nq() { return kNQ; }
int orc_nv() { return kNV; }

void orc_fk_f(int n, const float* q, float* xp, float* xq, float* xi) { fk_batch(n, q, xp, xq, xi); }
void orc_fk_recursive_f(int n, const float* q, float* xp, float* xq, float* xi) {
  for (int w = 0; w < n; ++w)
    fk_recursive(q + (long)w * kNQ, xp + (long)w * kNBody * 3, xq + (long)w * kNBody * 4, xi + (long)w * kNBody * 3);
}
void orc_fk_d(int n, const double* q, double* xp, double* xq, double* xi) { fk_batch(n, q, xp, xq, xi); }
void orc_bias_f(int n, const float* q, const float* v, float* S, float* b) { bias_batch(n, q, v, S, b); }
void orc_bias_d(int n, const double* q, const double* v, double* S, double* b) { bias_batch(n, q, v, S, b); }
void orc_mass_f(int n, const float* q, float* Mo) { mass_batch(n, q, Mo); }
void orc_mass_d(int n, const double* q, double* Mo) { mass_batch(n, q, Mo); }
void orc_solve_f(int n, const float* q, const float* Bdt, const float* x, float* y, int multi) { solve_batch(n, q, Bdt, x, y, multi); }
void orc_solve_d(int n, const double* q, const double* Bdt, const double* x, double* y, int multi) { solve_batch(n, q, Bdt, x, y, multi); }
void orc_qacc_f(int n, const float* q, const float* v, const float* tau, const float* Bdt, int pgs, float mu, float* qacc,
                int* ncon, int nthreads, int contact) { qacc_batch(n, q, v, tau, Bdt, pgs, mu, qacc, ncon, nthreads, contact); }
void orc_qacc_d(int n, const double* q, const double* v, const double* tau, const double* Bdt, int pgs, double mu,
                double* qacc, int* ncon, int nthreads, int contact) {
  qacc_batch(n, q, v, tau, Bdt, pgs, mu, qacc, ncon, nthreads, contact);
}
void orc_dyn_f(int n, float* q, float* v, const float* tau, int nsub, int contact, int damped, int guard, int pgs,
               float mu, float* qacc, int* ncon, int nthreads) {
  dyn_batch(n, q, v, tau, nsub, contact, damped, guard, pgs, mu, qacc, ncon, nthreads);
}
void orc_dyn_d(int n, double* q, double* v, const double* tau, int nsub, int contact, int damped, int guard, int pgs,
               double mu, double* qacc, int* ncon, int nthreads) {
  dyn_batch(n, q, v, tau, nsub, contact, damped, guard, pgs, mu, qacc, ncon, nthreads);
}
void orc_substep_f(int n, float* q, float* v, const float* target, int pgs, float mu, float* qacc, int* ncon,
                   int nthreads) { substep_batch(n, q, v, target, pgs, mu, qacc, ncon, nthreads); }
void orc_substep_d(int n, double* q, double* v, const double* target, int pgs, double mu, double* qacc, int* ncon,
                   int nthreads) { substep_batch(n, q, v, target, pgs, mu, qacc, ncon, nthreads); }

// Contact-solve intermediates of one state (fp32): A [nefc*nefc], b/f/R/aref [nefc], qacc_smooth.
int orc_qacc_debug_f(const float* q, const float* v, const float* tau, const float* Bdt, int pgs, float mu, float* qacc,
                     float* A, float* b, float* f, float* Rr, float* aref, float* qacc_s) {
  Frames<float> F; float S[kNV * 6];
  ContactDebug<float> dbg;
  fk(q, F.xpos, F.xquat, F.xipos);
  int nc = env_qacc(q, v, F, tau, Bdt, S, qacc, pgs, mu, &dbg);
  int nefc = 4 * nc;
  std::memcpy(A, dbg.A, sizeof(float) * nefc * nefc);
  std::memcpy(b, dbg.b, sizeof(float) * nefc);
  std::memcpy(f, dbg.f, sizeof(float) * nefc);
  std::memcpy(Rr, dbg.R_, sizeof(float) * nefc);
  std::memcpy(aref, dbg.aref, sizeof(float) * nefc);
  std::memcpy(qacc_s, dbg.qacc_smooth, sizeof(float) * kNV);
  return nc;
}

void orc_pgs_f(int n, const float* A, const float* b, float* f, int iters) { solve_pgs(A, b, f, n, iters); }
void orc_pgs_d(int n, const double* A, const double* b, double* f, int iters) { solve_pgs(A, b, f, n, iters); }
void orc_bdt_f(float* out) {
  for (int i = 0; i < kNV; ++i) out[i] = 0;
  for (int i = 0; i < kAct; ++i) out[act_dof[i]] = M<float>::dt * M<float>::act_kd[i];
}
void orc_bdt_d(double* out) {
  for (int i = 0; i < kNV; ++i) out[i] = 0;
  for (int i = 0; i < kAct; ++i) out[act_dof[i]] = M<double>::dt * M<double>::act_kd[i];
}
float orc_impedance_f(float pos) { return foot_impedance(pos); }
double orc_impedance_d(double pos) { return foot_impedance(pos); }

void orc_obs_f(int n, const float* qp, const float* qv, const float* pa, float* obs) {
  for (int w = 0; w < n; ++w) compute_obs(qp + (long)w * kNQ, qv + (long)w * kNV, pa + (long)w * kAct, obs + (long)w * kObs);
}

long orc_policy_params(int nl, const int* hid, int act) {
  PolicySpec ps{nl, {0, 0, 0, 0}, act};
  for (int l = 0; l < nl; ++l) ps.hid[l] = hid[l];
  return policy_params(ps);
}

void orc_mlp_f(int n, int nl, const int* hid, int act, const float* W, const float* x, float* mu, float* ls, float* v) {
  PolicySpec ps{nl, {0, 0, 0, 0}, act};
  for (int l = 0; l < nl; ++l) ps.hid[l] = hid[l];
  for (int w = 0; w < n; ++w) mlp_forward(W, ps, x + (long)w * kObs, mu + (long)w * kAct, ls + (long)w * kAct, v + w);
}

// One control step for n worlds, state in/out: the host-step (k_step) unit.
void orc_env_advance_f(int n, float* qp, float* qv, float* pa, int* steps, const float* act, const float* reset_noise,
                       int S, int pgs, float mu, float* rew, float* done, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 4)
  for (int w = 0; w < n; ++w) {
    float r; int d;
    env_advance(qp + (long)w * kNQ, qv + (long)w * kNV, pa + (long)w * kAct, &steps[w], act + (long)w * kAct,
                reset_noise + (long)w * kAct, S, pgs, mu, &r, &d);
    rew[w] = r; done[w] = (float)d;
  }
}

// Fused rollout for N worlds with pre-generated noise; state in/out; ncon_hist[9] optional.
void orc_rollout_f(int N, int H, int S, int pgs, float mu, float* qp, float* qv, float* pa, int* steps, const float* W,
                   int nl, const int* hid, int act, const float* mean, const float* var, const float* act_noise,
                   const float* reset_noise, float* O, float* A, float* LP, float* V, float* R, float* D, float* Vlast,
                   int* ncon_hist, int nthreads) {
  PolicySpec ps{nl, {0, 0, 0, 0}, act};
  for (int l = 0; l < nl; ++l) ps.hid[l] = hid[l];
  std::vector<int> hist((size_t)nthreads * 9, 0);
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
  for (int w = 0; w < N; ++w) {
    int tid = 0;
#ifdef _OPENMP
    tid = omp_get_thread_num();
#endif
    rollout_world(w, N, H, S, pgs, mu, qp, qv, pa, steps, W, ps, mean, var, act_noise, reset_noise, O, A, LP, V, R, D,
                  Vlast, &hist[(size_t)tid * 9]);
  }
  if (ncon_hist)
    for (int t = 0; t < nthreads; ++t)
      for (int k = 0; k < 9; ++k) ncon_hist[k] += hist[(size_t)t * 9 + k];
}

}  // extern "C"
