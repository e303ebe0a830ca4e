// queue.h -- the physics work items and the work queue shared by k_physics (g1env.hip) and
// k_rollout (rollout_kernel.hip): launch arguments, the hand-over between waves, and one item of a
// world pair's control step.
#pragma once
#include <hip/hip_runtime.h>

#include "physics.h"
#include "policy.h"
#include "rollout.h"

namespace g1k {

// ====================================================================== physics kernels
constexpr int kMaxChunks = 16;     // substep chunks per control step (work items of one pair)

struct PhysArgs {
  float* qp; float* qv; float* pa; int* steps; unsigned* rng;
  int N, S, pgs, K;                // K control steps per launch (same action buffer row t0 + k*astep)
  float mu;
  const float* act; int t0, astep; // actions [*, N, 29]; row t = t0 + k * astep
  const float* reset_noise;        // [*, N, 29] injected U(-1,1) or null (Philox)
  float* R; float* D; int rstep;   // outputs [*, N], row t0 + k * rstep
  float* obs;                      // [N][100] observation after the last control step, or null
  unsigned long long seed;
  unsigned long long* ncon_hist;   // [9] or null
  // work queue (k_physics below)
  unsigned* flags;                 // [pairs] chunks completed per world pair since the env was created
  unsigned fbase;                  // value every flag holds when this launch starts
  unsigned* qctr;                  // [2][kQueues] claim counters: this launch counts on row qpar and
  int qpar;                        //   clears row qpar ^ 1 for the next launch
  float* acc;                      // [N][32] per-lane energy sums of a control step split over items
  float* vxs;                      // [N] base x-velocity sum of a control step split over items
  int* qerr;                       // 1: a dependency wait exceeded kSpinLimit polls; 2: a wave of
                                   //   queue q ran outside XCD q while xlocal is set
  int xlocal;                      // queue q's waves all run on XCD q (checked at env creation)
  int nch;                         // work items (substep chunks) per pair and control step:
  int cst[kMaxChunks + 1];         //   chunk c = substeps [cst[c], cst[c + 1]), cst[nch] = S
  int nchl;                        // the same for the launch's last control step (k = K - 1)
  int cstl[kMaxChunks + 1];
  unsigned char* cflag;            // [N] or null: the world's contacts at the last substep of its
                                   //   last completed control step, 9 after an auto-reset (k_rollout's
                                   //   tile pairing)
};

constexpr int kPhysThreads = 64;   // one wave64 = two 32-lane world groups
static_assert(kPhysThreads == 64, "world_qacc orders its LDS hand-overs with wave_sync(): one wave per block");
constexpr int kXcds = 8;           // XCDs of the MI355X
constexpr int kQueues = 32;        // work queues, kQueues / kXcds per XCD (spreads the claim atomics)
constexpr unsigned kSpinLimit = 1u << 22;

__device__ __forceinline__ int xcc_id() { return (int)__builtin_amdgcn_s_getreg(20 | (0 << 6) | ((4 - 1) << 11)); }

// A value stored by another wave earlier in this launch: read from the L2, bypassing this CU's L1
// (an agent-scope load), so a line cached by an earlier item on this CU is never used.
template <class T>
__device__ __forceinline__ T ld_l2(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- work-queue hand-over between waves (k_physics, k_rollout)
// A value stored by another wave of the same launch is read from the L2 (ld_l2), the producer's
// stores are acknowledged before its flag moves, and flags only grow. The hardware places blocks on
// the 8 XCDs round-robin, so all waves of queue q share the L2 of XCD q mod 8 (xlocal, verified when
// the env is created and re-checked by every wave); the L2 is then the coherence point. Without
// xlocal the hand-over uses agent-scope release/acquire fences, which also write back and
// invalidate the L2 (correct on any placement, much slower).

// Wait until *flag >= want (wrap-safe). A wait that exceeds kSpinLimit polls sets qerr = 1 and
// returns: every item waited for was claimed earlier by a running wave, so a wait ends unless the
// hardware stalls; the error makes the next synchronising call exit.
__device__ __forceinline__ void wait_flag(const unsigned* flag, unsigned want, int* qerr, int xlocal) {
  unsigned spins = 0;
#pragma unroll 1
  for (;;) {
    const unsigned f = __builtin_amdgcn_readfirstlane(ld_l2(flag));
    if ((int)(f - want) >= 0) break;
    if (++spins > kSpinLimit) {
      if (threadIdx.x == 0) __hip_atomic_store(qerr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  if (xlocal) __asm__ volatile("" ::: "memory");
  else __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Publish the item's stores: every store acknowledged, then the flag moves to `value`.
__device__ __forceinline__ void release_flag(unsigned* flag, unsigned value, int xlocal) {
  __syncthreads();
  if (xlocal) __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  if (threadIdx.x == 0) __hip_atomic_store(flag, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One physics work item: world pair p (the two 32-lane groups of the wave), control step k of the
// launch, substeps [cst[c], cst[c + 1]) of it: PD torques, world_qacc, Euler; the last chunk of a
// control step adds the step's reward, termination and auto-reset (reference:
// src/g1_env.cu:118-212, the k_rollout substep loop :319-325). Every input a previous item or launch
// wrote is read from the L2 (the actions too: in k_rollout the policy items of the same launch
// write them).
__device__ __forceinline__ void physics_item(const PhysArgs& a, WorldLds& s, const LaneModel& L, int g, int l, int w,
                                             int k, int c, unsigned& hcnt) {
  const int ai = L.hinge ? L.b - 2 : 0;
  const SolveParams P{a.pgs, a.mu, true, true};
  const bool wvalid = w < a.N;
  const int wc = wvalid ? w : a.N - 1;   // an odd N's last group repeats world N - 1 and stores nothing

  LaneState st;
  const float* gq = a.qp + (long)wc * kNQ;
  const float* gv = a.qv + (long)wc * kNV;
#pragma unroll
  for (int m = 0; m < 7; ++m) st.bq[m] = ld_l2(gq + m);
#pragma unroll
  for (int m = 0; m < 6; ++m) st.bqd[m] = ld_l2(gv + m);
  st.jq = L.hinge ? ld_l2(gq + L.b + 5) : 0.f;
  st.jqd = L.hinge ? ld_l2(gv + L.b + 4) : 0.f;
  const int t = a.t0 + k * a.astep;
  const float act = L.hinge ? ld_l2(a.act + ((long)t * a.N + wc) * kAct + ai) : 0.f;
  // PD target = clamp(stand + 0.5 a) (reference: src/g1_env.cu:123-130)
  float target = fmaf_(0.5f, act, L.qstand);
  if (target < L.clo) target = L.clo;
  if (target > L.chi) target = L.chi;
  float vx_sum = 0.f, energy = 0.f;
  if (c > 0) {
    energy = ld_l2(a.acc + (long)wc * kGroup + l);
    vx_sum = ld_l2(a.vxs + wc);
  }
  const bool lastk = k == a.K - 1;   // the launch's last control step has a chunk table of its own
  const int nck = lastk ? a.nchl : a.nch;
  const int s0 = lastk ? a.cstl[c] : a.cst[c], s1 = lastk ? a.cstl[c + 1] : a.cst[c + 1];
  int nc_last = 0;   // the world's contacts at its last substep
#pragma unroll 1
  for (int sub = s0; sub < s1; ++sub) {
    float jtau = 0.f;
    if (L.hinge) {
      float pdt = fmaf_(-L.kd, st.jqd, L.kp * (target - st.jq));
      if (pdt < L.flo) pdt = L.flo;
      else if (pdt > L.fhi) pdt = L.fhi;
      jtau = pdt;
      energy += fabsf(pdt * st.jqd);
    }
    float bqacc[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, jqacc = 0.f;
    const int nc = world_qacc(l, s, st, jtau, P, bqacc, jqacc);
    hcnt += (l == nc && wvalid) ? 1u : 0u;
    nc_last = nc;
    integrate_lane(L, st, bqacc, jqacc, true);
    vx_sum += st.bqd[0];
  }
  if (c < nck - 1) {
    if (wvalid) {
      a.acc[(long)w * kGroup + l] = energy;
      if (l == 1) a.vxs[w] = vx_sum;
    }
  } else {
    // ---- reward / termination / auto-reset (reference: src/g1_env.cu:164-211), lane 1 decides
    float pa = L.hinge ? ld_l2(a.pa + (long)wc * kAct + ai) : 0.f;
    int step = ld_l2(a.steps + wc);
    unsigned rng = ld_l2(a.rng + wc);
    const float da = L.hinge ? act - pa : 0.f;
    float act_pen = gsum(da * da);
    const float energy_tot = gsum(energy);
    int d_flag = 0;
    float r = 0.f;
    if (l == 1) {
      const float vx = vx_sum / (float)a.S;
      const float height = st.bq[2];
      const float qx = st.bq[4], qy = st.bq[5];
      const float up = fmaf_(-2.f, fmaf_(qy, qy, qx * qx), 1.f);   // quat2mat(q)[2][2]
      const int alive = !(height < 0.45f || up < 0.5f);
      const float upc = up < 0.f ? 0.f : (up > 1.f ? 1.f : up);
      float vx_c = vx > 0.8f ? 0.8f : vx;
      if (vx_c < 0.f) vx_c = 0.f;
      const float r_vel = 1.0f * vx_c * upc;
      const float r_lat = -0.2f * fabsf(st.bqd[1]) - 0.05f * fabsf(st.bqd[5]);
      const float r_up = 0.3f * upc;
      const float r_h = -0.5f * fabsf(height - 0.78f);
      if (act_pen > 10.f) act_pen = 10.f;
      r = alive ? 1.0f + r_vel + r_lat + r_up + r_h - 0.005f * act_pen - 1e-4f * energy_tot : -5.0f;
      const int won = alive && st.bq[0] >= 5.0f;
      if (won) r += 50.0f;
      d_flag = (!alive || won || step + 1 >= 1000) ? 1 : 0;
    }
    d_flag = gshfl(d_flag, 1);
    step += 1;
    pa = act;
    if (d_flag) {
      const float u = a.reset_noise ? a.reset_noise[((long)t * a.N + wc) * kAct + ai]
                                    : rng_pm1(a.seed, wc, rng, kStreamReset, ai);
      if (L.hinge) { st.jq = L.qstand + 0.05f * u; st.jqd = 0.f; pa = 0.f; }
#pragma unroll
      for (int m = 0; m < 7; ++m) st.bq[m] = MF::qpos_stand[m];
#pragma unroll
      for (int m = 0; m < 6; ++m) st.bqd[m] = 0.f;
      step = 0;
    }
    rng += 1;
    if (wvalid) {
      // contacts at the last substep, or 9 after a reset to the stand pose (both feet down)
      if (a.cflag && l == 0) a.cflag[w] = (unsigned char)(d_flag ? 9 : nc_last);
      if (l == 1) {
        const long o = (long)(a.t0 + k * a.rstep) * a.N + w;
        a.R[o] = r;
        a.D[o] = (float)d_flag;
        a.steps[w] = step;
        a.rng[w] = rng;
      }
      if (L.hinge) a.pa[(long)w * kAct + ai] = pa;
      if (a.obs && k == a.K - 1) {
        // observation of the final state, each lane writing its own entries (same values as k_obs)
        float* o = a.obs + (long)w * kObs;
        if (l == 1) {
#pragma unroll
          for (int m = 0; m < 6; ++m) o[m] = st.bqd[m];
          const float qw = st.bq[3], qx = st.bq[4], qy = st.bq[5], qz = st.bq[6];
          o[6] = -(2.f * fmaf_(-qw, qy, qx * qz));
          o[7] = -(2.f * fmaf_(qw, qx, qy * qz));
          o[8] = -fmaf_(-2.f, fmaf_(qy, qy, qx * qx), 1.f);
        }
        if (L.hinge) { o[9 + ai] = st.jq; o[38 + ai] = st.jqd; o[67 + ai] = pa; }
        if (l == 0) { o[96] = 0.8f; o[97] = 0.f; o[98] = 0.f; o[99] = 0.f; }
      }
    }
  }
  if (wvalid) {
    float* oq = a.qp + (long)w * kNQ;
    float* ov = a.qv + (long)w * kNV;
    if (l == 1) {
#pragma unroll
      for (int m = 0; m < 7; ++m) oq[m] = st.bq[m];
#pragma unroll
      for (int m = 0; m < 6; ++m) ov[m] = st.bqd[m];
    }
    if (L.hinge) {
      oq[L.b + 5] = st.jq;
      ov[L.b + 4] = st.jqd;
    }
  }
}

// ====================================================================== the rollout in one launch
// k_rollout runs a whole g1_rollout: the physics items of k_physics for H control steps, and the
// policy of every control step on 16-world tiles (policy_tile). Tile u of queue q holds the pairs
// q + 32 (8 u + i), i < 8, so all its work stays on the queue's XCD.
// Claim order within a queue (nq pairs, ntq tiles, nch substep chunks per control step, nchl in
// the last one):
//   P(0, all tiles), then C(t, c, all pairs) for t < H, c < (t < H - 1 ? nch : nchl),
// where P(0, u) is the policy of step 0 on tile u and C(t, c, p) chunk c of pair p's step t. The
// policy of a later step is not claimed: the wave that completes a tile's last pair of step t (the
// tile's completion count, raised by every pair's last chunk after its release, reaches the tile's
// pair count; that wave clears it) runs P(t + 1, u) at once, so no wave waits for a tile to complete;
// P(H, u) computes the bootstrap value. Waits: C(t, c > 0, p) on C(t, c - 1, p) (the pair's flag,
// claimed earlier); C(t, 0, p) on P(t, u(p)) (the tile's flag), which either was claimed earlier or
// runs in the wave that completed the tile's step t - 1, a running wave. So every wait ends.
struct RolloutArgs {
  PhysArgs ph;              // K = H control steps, actions from A
  TileArgs po;
  unsigned* tflags;         // [kQueues * tiles per queue] policy steps completed per tile
  unsigned tbase;           // value every tile flag holds when this launch starts
  unsigned* tcount;         // [kQueues * tiles per queue] pairs of a tile done with the current step
                            // (zero between launches)
  unsigned long long* tperm;   // [kQueues * tiles per queue] the tile's pairing of the current step:
                               //   nibble 2 i + g = the world slot that group g of pair slot i runs
};

// A kernel's by-value argument block (its only argument, at offset 0 of the kernarg segment),
// re-read where it is used: the opaque copy of the segment address keeps the compiler from
// loading every field once at the top and holding them across the work loop, in scalar
// registers spilled to vector lanes and in copies in vector registers the physics needs.
template <class T>
__device__ __forceinline__ const T& kernarg_reread() {
  typedef const __attribute__((address_space(4))) T* KargPtr;
  KargPtr p = (KargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  __asm__ volatile("" : "+s"(p));
  return *(const T*)p;
}

// Enqueue the one-launch rollout kernel on the null stream (rollout_kernel.hip).
void launch_rollout_kernel(const RolloutArgs& ra, int grid);
// k_rollout's function handles (occupancy report): the register-resident policy tile, or the wide one.
const void* rollout_kernel_fn(bool wide);

}  // namespace g1k
