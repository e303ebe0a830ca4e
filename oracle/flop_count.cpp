// flop_count.cpp -- the oracle's algorithm instantiated on an operation-counting scalar. TEST
// INFRASTRUCTURE ONLY (built into oracle/libg1flops.so by oracle/Makefile; loaded by tests/, which
// derive and check the FLOP table of g1.cu_amd/roofline.py with it; never by the product path).
//
// flc::F wraps a float and counts every arithmetic operation performed on it: additions and
// subtractions, multiplications, fused multiply-adds, divisions, square roots, comparisons and
// transcendental calls. g1_oracle.cpp is included unchanged: its templates are instantiated with
// R = flc::F, the model tables are copied into ModelT<flc::F>, and the oracle's math helpers
// (fma_, sqrt_, sin_, ...) resolve to the counting overloads below by argument-dependent lookup.
// The forward-kinematics compositions, which the oracle runs in fp64, are counted as flc::F too.
//
// Exports: flc_substep (one env substep of one world: FK, PD torque, contact detection and solve,
// Euler and position integration) and flc_step_overhead (the per-control-step work outside the
// substeps: PD targets, reward, termination), each returning the operation counts.
#include <cmath>
#include <cstring>

#include "../g1.cu_amd/csrc/g1_model_tables.h"

namespace flc {

struct Counts {
  unsigned long long add, mul, fma, div, sqrt, cmp, trans;
};
static Counts cnt;   // single-threaded use (the entry points run one world on the calling thread)

struct F {
  float v;
  F() = default;
  constexpr F(float x) : v(x) {}
  constexpr F(double x) : v((float)x) {}
  constexpr F(int x) : v((float)x) {}
  explicit operator double() const { return v; }
  explicit operator float() const { return v; }
};

inline F operator+(F a, F b) { ++cnt.add; return F(a.v + b.v); }
inline F operator-(F a, F b) { ++cnt.add; return F(a.v - b.v); }
inline F operator*(F a, F b) { ++cnt.mul; return F(a.v * b.v); }
inline F operator/(F a, F b) { ++cnt.div; return F(a.v / b.v); }
inline F operator-(F a) { return F(-a.v); }   // a sign flip, not an arithmetic operation
inline F& operator+=(F& a, F b) { a = a + b; return a; }
inline F& operator-=(F& a, F b) { a = a - b; return a; }
inline F& operator*=(F& a, F b) { a = a * b; return a; }
inline F& operator/=(F& a, F b) { a = a / b; return a; }
inline bool operator<(F a, F b) { ++cnt.cmp; return a.v < b.v; }
inline bool operator>(F a, F b) { ++cnt.cmp; return a.v > b.v; }
inline bool operator<=(F a, F b) { ++cnt.cmp; return a.v <= b.v; }
inline bool operator>=(F a, F b) { ++cnt.cmp; return a.v >= b.v; }
inline bool operator==(F a, F b) { ++cnt.cmp; return a.v == b.v; }
inline bool operator!=(F a, F b) { ++cnt.cmp; return a.v != b.v; }

// the oracle's math helpers, found by argument-dependent lookup ahead of its own templates
inline F fma_(F a, F b, F c) { ++cnt.fma; return F(std::fma(a.v, b.v, c.v)); }
inline F sqrt_(F x) { ++cnt.sqrt; return F(std::sqrt(x.v)); }
inline F rsqrt_(F x) { ++cnt.sqrt; ++cnt.div; return F(1.0f / std::sqrt(x.v)); }
inline F fabs_(F x) { return F(std::fabs(x.v)); }
inline bool isfinite_(F x) { ++cnt.cmp; return std::isfinite(x.v); }
inline F sin_(F x) { ++cnt.trans; return F((float)std::sin((double)x.v)); }
inline F cos_(F x) { ++cnt.trans; return F((float)std::cos((double)x.v)); }
inline F pow_(F x, F y) { ++cnt.trans; return F((float)std::pow((double)x.v, (double)y.v)); }
inline F tanh_(F x) { ++cnt.trans; return F(std::tanh(x.v)); }
inline F expm1_(F x) { ++cnt.trans; return F(std::expm1(x.v)); }
inline F exp_(F x) { ++cnt.trans; return F(std::exp(x.v)); }
inline unsigned long long bits_of(F x) { unsigned u; std::memcpy(&u, &x.v, 4); return u; }

}  // namespace flc

namespace g1 {
// The fp32 model tables as counting scalars (filled by init_tables before any count).
template <> struct ModelT<flc::F> {
  static flc::F dt, foot_radius, foot_mu, foot_impratio;
  static flc::F gravity[3], body_pos[93], body_quat[124], body_ipos[93], body_iquat[124], body_mass[31];
  static flc::F body_inertia[93], jnt_axis[90], jnt_pos[90], dof_armature[35], qpos0[36], qpos_stand[36];
  static flc::F foot_lpos[24], foot_solref[2], foot_solimp[5], foot_invweight0[8];
  static flc::F act_kp[29], act_kd[29], act_ctrl_lo[29], act_ctrl_hi[29], act_frc_lo[29], act_frc_hi[29];
};
}  // namespace g1

#define G1_FLC_TABLES(X)                                                                             \
  X(gravity) X(body_pos) X(body_quat) X(body_ipos) X(body_iquat) X(body_mass) X(body_inertia)        \
  X(jnt_axis) X(jnt_pos) X(dof_armature) X(qpos0) X(qpos_stand) X(foot_lpos) X(foot_solref)          \
  X(foot_solimp) X(foot_invweight0) X(act_kp) X(act_kd) X(act_ctrl_lo) X(act_ctrl_hi) X(act_frc_lo) \
  X(act_frc_hi)

namespace g1 {
flc::F ModelT<flc::F>::dt, ModelT<flc::F>::foot_radius, ModelT<flc::F>::foot_mu, ModelT<flc::F>::foot_impratio;
#define G1_FLC_DEF(name) flc::F ModelT<flc::F>::name[sizeof(ModelT<float>::name) / sizeof(float)];
G1_FLC_TABLES(G1_FLC_DEF)
#undef G1_FLC_DEF
}  // namespace g1

static void init_tables() {
  using MFt = g1::ModelT<float>;
  using MC = g1::ModelT<flc::F>;
  MC::dt = MFt::dt; MC::foot_radius = MFt::foot_radius; MC::foot_mu = MFt::foot_mu;
  MC::foot_impratio = MFt::foot_impratio;
#define G1_FLC_COPY(name)                                                                      \
  static_assert(sizeof(MC::name) / sizeof(flc::F) == sizeof(MFt::name) / sizeof(float), #name); \
  for (size_t i = 0; i < sizeof(MFt::name) / sizeof(float); ++i) MC::name[i] = flc::F(MFt::name[i]);
  G1_FLC_TABLES(G1_FLC_COPY)
#undef G1_FLC_COPY
}

#include "g1_oracle.cpp"

namespace orc {
template <> struct ComposePrec<flc::F> { using type = flc::F; };   // count the fp64 compositions too
template <> struct FkComposeIdentity<flc::F> { static constexpr bool value = false; };   // padding, not work
}

static void out_counts(double* out7) {
  const flc::Counts& c = flc::cnt;
  out7[0] = (double)c.add; out7[1] = (double)c.mul; out7[2] = (double)c.fma; out7[3] = (double)c.div;
  out7[4] = (double)c.sqrt; out7[5] = (double)c.cmp; out7[6] = (double)c.trans;
}

extern "C" {

// One env substep of one world from (qp [36], qv [35]) toward PD targets target [29], pgs sweeps,
// friction mu; ref_order 1 counts the reference's summation association, 0 the kernel's. Returns
// the contact count; out7 = {add/sub, mul, fma, div, sqrt, compare, transcendental}.
int flc_substep(const float* qp, const float* qv, const float* target, int pgs, float mu, int ref_order, double* out7) {
  init_tables();
  using flc::F;
  F q[orc::kNQ], v[orc::kNV], tg[orc::kAct];
  for (int i = 0; i < orc::kNQ; ++i) q[i] = F(qp[i]);
  for (int i = 0; i < orc::kNV; ++i) v[i] = F(qv[i]);
  for (int i = 0; i < orc::kAct; ++i) tg[i] = F(target[i]);
  orc::g_ref_order = ref_order ? 1 : 0;
  int nc = 0;
  flc::cnt = flc::Counts{};
  ::substep_batch<F>(1, q, v, tg, pgs, F(mu), nullptr, &nc, 1);
  out_counts(out7);
  orc::g_ref_order = 0;
  return nc;
}

// The work of one control step outside its substeps (PD targets from the action, reward,
// termination, reset bookkeeping): env_advance with zero substeps on a standing world.
void flc_step_overhead(int ref_order, double* out7) {
  init_tables();
  using flc::F;
  F q[orc::kNQ], v[orc::kNV], pa[orc::kAct], a[orc::kAct], noise[orc::kAct];
  for (int i = 0; i < orc::kNQ; ++i) q[i] = g1::ModelT<F>::qpos_stand[i];
  for (int i = 0; i < orc::kNV; ++i) v[i] = F(0.f);
  for (int i = 0; i < orc::kAct; ++i) { pa[i] = F(0.f); a[i] = F(0.1f); noise[i] = F(0.f); }
  orc::g_ref_order = ref_order ? 1 : 0;
  int step = 0, done = 0;
  F r;
  flc::cnt = flc::Counts{};
  orc::env_advance<F>(q, v, pa, &step, a, noise, 0, 8, F(0.6f), &r, &done);
  out_counts(out7);
  orc::g_ref_order = 0;
}

}  // extern "C"
