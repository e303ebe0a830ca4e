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
    // The tile's pairing for step t: its 16 slots in descending order of their worlds' contact
    // counts at the last substep of step t - 1 (a stable sort; 9 after an auto-reset), so that
    // consecutive slots form the pairs: a wave runs the contact pipeline when either of its worlds
    // has contacts, at a cost that grows with the larger count, and the counts at the end of a step
    // predict the next (fixed pairs run it in ~70% of config 3's pair-substeps, these ~63%). Which
    // two worlds share a wave changes no result. Step 0 and partial tiles keep the fixed pairs
    // (slot 2 i + g runs group g of pair slot i).
    if (rb.tperm) {
      unsigned long long pm = 0xFEDCBA9876543210ull;
      if (t > 0 && np == kTilePairs && tile_world(qq, u, 2 * kTilePairs - 1, kQueues) < b.N) {
        const int key = min((int)ld_l2(b.cflag + w), 9);
        const unsigned mask16 = (1u << jw) - 1u;
        // position = slots with a larger key + earlier slots with the same key (lanes 0..15 hold
        // slots 0..15; the other lanes repeat them)
        int pos = 0;
#pragma unroll
        for (int v = 0; v <= 9; ++v) {
          const unsigned bv = (unsigned)__ballot(key == v) & 0xFFFFu;
          pos += v > key ? __popc(bv) : (v == key ? __popc(bv & mask16) : 0);
        }
        unsigned lo = pos < 8 ? (unsigned)jw << (4 * pos) : 0u, hi = pos >= 8 ? (unsigned)jw << (4 * (pos - 8)) : 0u;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          lo |= __shfl_xor(lo, o, 16);
          hi |= __shfl_xor(hi, o, 16);
        }
        pm = ((unsigned long long)hi << 32) | lo;
      }
      if (threadIdx.x == 0) rb.tperm[qq + kQueues * u] = pm;
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
      // this group's world: slot (pairing nibble 2 i + g) of the pair's tile, i = m mod 8
      const RolloutArgs& rb = kernarg_reread<RolloutArgs>();
      int w = 2 * p + g;
      if (rb.tperm) {
        const unsigned long long pm = ld_l2(rb.tperm + qc + kQueues * u);
        w = tile_world(qc, u, (int)((pm >> (4 * (2 * (m % kTilePairs) + g))) & 15ull), kQueues);
      }
      physics_item(rb.ph, s, L, g, l, w, t, c, hcnt);
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
