// rollout_kernel.hip -- k_rollout, the whole g1_rollout in one persistent launch (the scheme and
// its argument block are described in queue.h). Its own translation unit, so that it alone takes
// the wavefront-fence phase boundaries (G1_PHASE_FENCE below).
#include <hip/hip_runtime.h>

#define G1_PHASE_FENCE   // world_qacc's phase boundaries as wavefront fences (see wave_sync)
#include "queue.h"

namespace g1k {

// LDS of a k_rollout block: the two worlds' physics scratch, or a policy tile's scratch
constexpr size_t kRolloutLds = 2 * sizeof(WorldLds) > sizeof(float) * kTileLds
                                   ? 2 * sizeof(WorldLds) : sizeof(float) * kTileLds;

// kWide: the policy items run the wide tile (policy_tile_wide) instead of the register-resident
// 256-256 tile; two instantiations, so that each keeps its own register allocation (the physics
// items of the narrow kernel are not scheduled around the wide tile's accumulators).
template <bool kWide>
__global__ void __launch_bounds__(kPhysThreads) k_rollout(RolloutArgs ra) {
  __shared__ __align__(16) unsigned char lds_raw[kRolloutLds];
  WorldLds* lds = reinterpret_cast<WorldLds*>(lds_raw);
  const PhysArgs& a = ra.ph;
  const int g = group_id(), l = group_lane();
  WorldLds& s = lds[g];
  const int q = blockIdx.x % kQueues;
  if (blockIdx.x == 0 && threadIdx.x < kQueues) a.qctr[(a.qpar ^ 1) * kQueues + threadIdx.x] = 0u;
  const int npairs = (a.N + 1) >> 1;
  const int nch = a.nch, H = a.K;
  int qc = q;
  unsigned nq = 0, ntq = 0, nitems = 0;
  unsigned* ctr = nullptr;
  auto set_queue = [&](int qq) {
    nq = npairs > qq ? (unsigned)((npairs - qq + kQueues - 1) / kQueues) : 0u;
    ntq = (nq + kTilePairs - 1) / kTilePairs;
    nitems = nq ? ntq + (H > 0 ? (unsigned)((H - 1) * nch + a.nchl) * nq : 0u) : 0u;
    ctr = a.qctr + a.qpar * kQueues + qq;
  };
  set_queue(q);
  unsigned hcnt = 0;
  if (a.xlocal && threadIdx.x == 0 && xcc_id() != q % kXcds)
    __hip_atomic_store(a.qerr, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float* scratch_lds = reinterpret_cast<float*>(lds_raw);
  // policy of step t on tile u of queue qq (its np pairs complete through step t - 1)
  auto policy = [&](int qq, int u, int np, int t) {
    const int jw = threadIdx.x & 15;
    const int w = tile_world(qq, u, jw, kQueues);
    const bool valid = (jw >> 1) < np && w < a.N;
    const auto ld = [](const auto* ptr) { return ld_l2(ptr); };
    const RolloutArgs& rb = kernarg_reread<RolloutArgs>();
    const PhysArgs& b = rb.ph;
    if constexpr (kWide) {
      // this block's two activation buffers
      float* scr = rb.po.scr + (long)blockIdx.x * 2 * rb.po.wl.maxT * 256;
      if (rb.po.wl.act == 0)
        policy_tile_wide<0>(rb.po, b.qp, b.qv, b.pa, b.rng, b.seed, b.N, t, w, valid, scratch_lds, scr, ld);
      else
        policy_tile_wide<1>(rb.po, b.qp, b.qv, b.pa, b.rng, b.seed, b.N, t, w, valid, scratch_lds, scr, ld);
    } else if (rb.po.tl.act == 0) {
      policy_tile<0>(rb.po, b.qp, b.qv, b.pa, b.rng, b.seed, b.N, t, w, valid, scratch_lds, ld);
    } else {
      policy_tile<1>(rb.po, b.qp, b.qv, b.pa, b.rng, b.seed, b.N, t, w, valid, scratch_lds, ld);
    }
    release_flag(ra.tflags + qq + kQueues * u, ra.tbase + (unsigned)t + 1u, a.xlocal);
  };

#pragma unroll 1
  for (;;) {
    unsigned mine = 0;
    if (threadIdx.x == 0) mine = atomicAdd(ctr, 1u);
    const unsigned it = __builtin_amdgcn_readfirstlane(mine);
    if (it >= nitems) {
      qc = qc + kXcds < kQueues ? qc + kXcds : qc + kXcds - kQueues;
      if (qc == q) break;
      set_queue(qc);
      continue;
    }
    // the policy this wave runs after its item, if any (one call site: one copy of its code)
    int pol_u = -1, pol_np = 0, pol_t = 0;
    if (it < ntq) {
      pol_u = (int)it;
      pol_np = (int)min((unsigned)kTilePairs, nq - kTilePairs * it);
    } else {
    // chunk index jj of the pair within the launch (its flag counts completed chunks)
    const unsigned r = it - ntq, nreg = (unsigned)((H - 1) * nch) * nq;
    int jj, m, t, c;
    if (r < nreg) {
      jj = (int)(r / nq); m = (int)(r - (unsigned)jj * nq);
      t = jj / nch; c = jj - t * nch;
    } else {
      const unsigned rl = r - nreg;
      c = (int)(rl / nq); m = (int)(rl - (unsigned)c * nq);
      t = H - 1; jj = (H - 1) * nch + c;
    }
    const int nck = t == H - 1 ? a.nchl : nch;
    const int p = qc + kQueues * m;
    const int u = m / kTilePairs;
    if (c > 0) wait_flag(a.flags + p, a.fbase + (unsigned)jj, a.qerr, a.xlocal);
    else wait_flag(ra.tflags + qc + kQueues * u, ra.tbase + (unsigned)t + 1u, a.qerr, a.xlocal);
    {
      // the lane's model constants, formed here (opaque lane index) rather than held across items
      int lo = l;
      __asm__ volatile("" : "+v"(lo));
      const LaneModel L = lane_model(lo);
      physics_item(kernarg_reread<RolloutArgs>().ph, s, L, g, l, p, t, c, hcnt);
    }
    release_flag(a.flags + p, a.fbase + (unsigned)jj + 1u, a.xlocal);
    if (c == nck - 1) {
      // this pair's step t is complete: count it for the tile; the wave completing the tile runs
      // the tile's policy of step t + 1
      const int np = (int)min((unsigned)kTilePairs, nq - kTilePairs * (unsigned)u);
      unsigned old = 0;
      if (threadIdx.x == 0)
        old = __hip_atomic_fetch_add(ra.tcount + qc + kQueues * u, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      old = __builtin_amdgcn_readfirstlane(old);
      if (old + 1u == (unsigned)np) {
        // no pair of the tile counts again before this policy's flag release: clear the count here
        if (threadIdx.x == 0)
          __hip_atomic_store(ra.tcount + qc + kQueues * u, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (!a.xlocal) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        pol_u = u; pol_np = np; pol_t = t + 1;
      }
    }
    }
    if (pol_u >= 0) policy(qc, pol_u, pol_np, pol_t);
  }
  if (a.ncon_hist && l < 9 && hcnt) atomicAdd(&a.ncon_hist[l], (unsigned long long)hcnt);
}

void launch_rollout_kernel(const RolloutArgs& ra, int grid) {
  if (ra.po.wide) hipLaunchKernelGGL(k_rollout<true>, dim3((unsigned)grid), dim3(kPhysThreads), 0, 0, ra);
  else hipLaunchKernelGGL(k_rollout<false>, dim3((unsigned)grid), dim3(kPhysThreads), 0, 0, ra);
}

const void* rollout_kernel_fn(bool wide) { return wide ? (const void*)k_rollout<true> : (const void*)k_rollout<false>; }

}  // namespace g1k
