// g1env.hip -- MI355X (gfx950) implementation of g1.cu's batched G1 environment and fused PPO
// rollout behind the reference's libg1env.so C ABI (reference: src/g1_env.cu:361-476).
//
// Rollout structure: g1_rollout enqueues, on the null stream and without any host sync,
//   pack(W) -> [policy(t) -> physics(t)] for t < H -> policy(H) (bootstrap value)
// policy(t): obs -> frozen normalisation -> MLP on fp32 MFMA over 32-world tiles -> sampling;
// physics(t): S substeps of FK -> PD -> world_qacc -> Euler on 32-lane world groups, then reward,
// termination and auto-reset. Trajectory tensors O/A/LP/V/R/D/Vlast are caller-owned device
// buffers written in place, exactly as the reference's k_rollout does (src/g1_env.cu:278-338).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/g1env.h"
#include "physics.h"
#include "policy.h"
#include "rollout.h"

using namespace g1k;

#define HIPCHECK(call)                                                                          \
  do {                                                                                          \
    hipError_t e_ = (call);                                                                     \
    if (e_ != hipSuccess) {                                                                     \
      fprintf(stderr, "g1env HIP error %s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      exit(1);                                                                                  \
    }                                                                                           \
  } while (0)

static void fail(const char* msg) {
  fprintf(stderr, "g1env: %s\n", msg);
  exit(1);
}

#include "queue.h"

constexpr int kStepChunks = 4;     // host-step copies between pageable and pinned memory, pipelined

// One physics launch advances every world pair (the two 32-lane groups of a wave64) by K control
// steps of S substeps (physics_item).
//
// The work is cut into items (world pair, chunk of substeps of one control step) that
// persistent waves claim from a queue, instead of one block per pair for the whole launch: a pair
// with contacts costs 2-3x a contact-free one, which contact state one control step earlier does
// not predict, and with whole-launch blocks the heavy blocks dispatched last keep a few SIMDs busy
// long after the rest have drained. Items are claimed in chunk-major order, so every pair advances
// about equally and the launch ends within about one item of its average.
//
// Queue q serves the pairs p = q (mod 32) and is claimed by the blocks with blockIdx = q (mod 32);
// a block whose queue is empty goes on with the other queues of its XCD (q + 8, q + 16, q + 24 mod
// 32), which evens out queues that drew more pairs with contacts. Item (p, j) needs item (p, j - 1),
// which was claimed earlier from the same queue by a wave that is running, so a wait always ends;
// the pair's flag counts its completed items.
__global__ void __launch_bounds__(kPhysThreads) k_physics(PhysArgs a) {
  __shared__ WorldLds lds[2];
  const int g = group_id(), l = group_lane();
  WorldLds& s = lds[g];
  const LaneModel L = lane_model(l);
  const int q = blockIdx.x % kQueues;
  if (blockIdx.x == 0 && threadIdx.x < kQueues) a.qctr[(a.qpar ^ 1) * kQueues + threadIdx.x] = 0u;
  const int npairs = (a.N + 1) >> 1;
  const int nch = a.nch;
  // items of a pair: nch per control step, nchl in the launch's last one (its own chunk table)
  const unsigned per_pair = (unsigned)((a.K - 1) * nch + a.nchl), nreg = (unsigned)((a.K - 1) * nch);
  // queue qc being drained: the block's own, then the other queues of its XCD (same L2, so the
  // hand-over holds; every item waited for was claimed earlier by a running wave)
  int qc = q;
  unsigned nq, nitems;
  unsigned* ctr;
  auto set_queue = [&](int qq) {
    nq = npairs > qq ? (unsigned)((npairs - qq + kQueues - 1) / kQueues) : 0u;
    nitems = nq * per_pair;
    ctr = a.qctr + a.qpar * kQueues + qq;
  };
  set_queue(q);
  unsigned hcnt = 0;   // lane q < 9 counts substeps with q contacts
  if (a.xlocal && threadIdx.x == 0 && xcc_id() != q % kXcds)
    __hip_atomic_store(a.qerr, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

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
    const int j = (int)(it / nq);
    const int p = qc + kQueues * (int)(it - (unsigned)j * nq);
    const int k = (unsigned)j < nreg ? j / nch : a.K - 1;
    const int c = j - k * nch;
    if (j > 0) wait_flag(a.flags + p, a.fbase + (unsigned)j, a.qerr, a.xlocal);
    physics_item(kernarg_reread<PhysArgs>(), s, L, g, l, 2 * p + g, k, c, hcnt);
    release_flag(a.flags + p, a.fbase + (unsigned)j + 1u, a.xlocal);
  }
  if (a.ncon_hist && l < 9 && hcnt) atomicAdd(&a.ncon_hist[l], (unsigned long long)hcnt);
}

// Pack torch-order weights (W0, b0, W1, b1, Wmu, bmu, Wv, bv, log_std) into the tile layout.
struct TilePackArgs {
  const float* W; const float* mean; const float* var; float* Wt; TileLayout tl; int h0, h1;
};
__global__ void k_pack_tiles(TilePackArgs a) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const TileLayout& T = a.tl;
  if (idx >= T.total) return;
  const long oW0 = 0, ob0 = oW0 + (long)a.h0 * kObs, oW1 = ob0 + a.h0, ob1 = oW1 + (long)a.h1 * a.h0,
             oWmu = ob1 + a.h1, obmu = oWmu + (long)kAct * a.h1, oWv = obmu + kAct, obv = oWv + a.h1, ols = obv + 1;
  float v = 0.f;
  if (idx >= T.nrm_off) {
    // normalisation constants of feature 4 s + g at [c][g][s] (the divisor as the split policy's)
    const int rel = (int)(idx - T.nrm_off), c = rel / (4 * kObsSteps), r = rel - c * 4 * kObsSteps;
    const int g = r / kObsSteps, k = 4 * (r - g * kObsSteps) + g;
    if (k < kObs) {
      const float dv = sqrtf(a.var[k] + 1e-8f);
      v = c == 0 ? a.mean[k] : (c == 1 ? dv : rcp_rn(dv));
    } else {
      v = c == 0 ? 0.f : 1.f;
    }
  } else if (idx >= T.ls_off) {
    const int i = (int)(idx - T.ls_off);
    v = i < kAct ? a.W[ols + i] : 0.f;
  } else {
    int Ly = 0;
    while (Ly < 2 && idx >= T.woff[Ly + 1]) ++Ly;
    const int kin = Ly == 0 ? kObs : (Ly == 1 ? a.h0 : a.h1);
    if (idx >= T.boff[Ly]) {
      const int row = (int)(idx - T.boff[Ly]);
      if (Ly == 0) v = row < a.h0 ? a.W[ob0 + row] : 0.f;
      else if (Ly == 1) v = row < a.h1 ? a.W[ob1 + row] : 0.f;
      else v = row < kAct ? a.W[obmu + row] : (row == kAct ? a.W[obv] : 0.f);
    } else {
      const long rel = idx - T.woff[Ly];
      const int e = (int)(rel & 3), lane = (int)((rel >> 2) & 63);
      const long rq = rel >> 8;
      const int qd = (int)(rq % T.nQ[Ly]), ot = (int)(rq / T.nQ[Ly]);
      const int row = 16 * ot + (lane & 15), k = tile_kappa(Ly, 4 * qd + e, lane >> 4);
      if (k < kin) {
        if (Ly == 0) v = row < a.h0 ? a.W[oW0 + (long)row * kObs + k] : 0.f;
        else if (Ly == 1) v = row < a.h1 ? a.W[oW1 + (long)row * a.h0 + k] : 0.f;
        else v = row < kAct ? a.W[oWmu + (long)row * a.h1 + k] : (row == kAct ? a.W[oWv + k] : 0.f);
      }
    }
  }
  a.Wt[idx] = v;
}

// Pack torch-order weights (W0, b0, .., Wmu, bmu, Wv, bv, log_std) of a policy of nl hidden layers
// into the wide tile's layout (WideLayout).
struct WidePackArgs {
  const float* W; const float* mean; const float* var; float* Wt; WideLayout wl; int hid[kMaxLayers];
};
__global__ void k_pack_wide(WidePackArgs a) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const WideLayout& T = a.wl;
  if (idx >= T.total) return;
  float v = 0.f;
  if (idx >= T.nrm_off) {
    // normalisation constants of feature 4 s + g at [c][g][s] (the divisor as the split policy's)
    const int rel = (int)(idx - T.nrm_off), c = rel / (4 * kObsSteps), r = rel - c * 4 * kObsSteps;
    const int g = r / kObsSteps, k = 4 * (r - g * kObsSteps) + g;
    if (k < kObs) {
      const float dv = sqrtf(a.var[k] + 1e-8f);
      v = c == 0 ? a.mean[k] : (c == 1 ? dv : rcp_rn(dv));
    } else {
      v = c == 0 ? 0.f : 1.f;
    }
  } else {
    // torch offsets of the layers before Ly, and of the head's parts
    int Ly = 0;
    while (Ly < T.nl && idx >= T.woff[Ly + 1]) ++Ly;
    long oW = 0;
    int in = kObs;
    for (int q = 0; q < T.nl && q < Ly; ++q) { oW += (long)a.hid[q] * in + a.hid[q]; in = a.hid[q]; }
    if (idx >= T.ls_off) {
      long oh = 0;
      int hin = kObs;
      for (int q = 0; q < T.nl; ++q) { oh += (long)a.hid[q] * hin + a.hid[q]; hin = a.hid[q]; }
      const int i = (int)(idx - T.ls_off);
      v = i < kAct ? a.W[oh + (long)kAct * hin + kAct + hin + 1 + i] : 0.f;
    } else {
      const bool head = Ly == T.nl;
      const long oWv = oW + (long)kAct * in + kAct;   // head: Wv, then bv after it
      if (idx >= T.boff[Ly]) {
        const int row = (int)(idx - T.boff[Ly]);
        if (!head) v = row < a.hid[Ly] ? a.W[oW + (long)a.hid[Ly] * in + row] : 0.f;
        else v = row < kAct ? a.W[oW + (long)kAct * in + row] : (row == kAct ? a.W[oWv + in] : 0.f);
      } else {
        const long rel = idx - T.woff[Ly];
        const int e = (int)(rel & 3), lane = (int)((rel >> 2) & 63);
        const long rq = rel >> 8;
        const int qd = (int)(rq % T.nQ[Ly]), ot = (int)(rq / T.nQ[Ly]);
        const int row = 16 * ot + (lane & 15), k = tile_kappa(Ly, 4 * qd + e, lane >> 4);
        if (k < in) {
          if (!head) v = row < a.hid[Ly] ? a.W[oW + (long)row * in + k] : 0.f;
          else v = row < kAct ? a.W[oW + (long)row * in + k] : (row == kAct ? a.W[oWv + k] : 0.f);
        }
      }
    }
  }
  a.Wt[idx] = v;
}

// XCD of each block of a grid shaped like k_physics' (placement check of the work queue)
__global__ void __launch_bounds__(kPhysThreads) k_xcc(int* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// ---- probes: the same world_qacc device code on caller-given states (parity harnesses)
struct ProbeArgs {
  int n, mode;            // mode 0: qacc only; 1: env substeps (PD from targets, integrate);
                          // 2: substeps driven by tau (integrate)
  float* qp; float* qv;   // [n][36], [n][35]; updated in place by modes 1 and 2
  const float* tau;       // modes 0, 2: [n][35] generalized force on the hinge dofs (base entries ignored)
  const float* target;    // mode 1: [n][29] PD joint targets
  float* qacc; int* ncon; // [n][35], [n]
  int pgs, damped, contact, guard, nsub;
  float mu;
};

__global__ void __launch_bounds__(kPhysThreads) k_probe(ProbeArgs a) {
  __shared__ WorldLds lds[2];
  const int g = group_id(), l = group_lane();
  const int w = blockIdx.x * 2 + g;
  const bool wvalid = w < a.n;
  const int wc = wvalid ? w : a.n - 1;
  WorldLds& s = lds[g];
  const LaneModel L = lane_model(l);
  LaneState st;
  const float* gq = a.qp + (long)wc * kNQ;
  const float* gv = a.qv + (long)wc * kNV;
#pragma unroll
  for (int k = 0; k < 7; ++k) st.bq[k] = gq[k];
#pragma unroll
  for (int k = 0; k < 6; ++k) st.bqd[k] = gv[k];
  st.jq = L.hinge ? gq[L.b + 5] : 0.f;
  st.jqd = L.hinge ? gv[L.b + 4] : 0.f;
  const SolveParams P{a.pgs, a.mu, a.damped != 0, a.contact != 0};
  float bqacc[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, jqacc = 0.f;
  int nc = 0;
#pragma unroll 1
  for (int sub = 0; sub < a.nsub; ++sub) {
    float jtau = 0.f;
    if (L.hinge) {
      if (a.mode != 1) jtau = a.tau[(long)wc * kNV + L.b + 4];
      else {
        const float tg = a.target[(long)wc * kAct + L.b - 2];
        float pdt = fmaf_(-L.kd, st.jqd, L.kp * (tg - st.jq));
        if (pdt < L.flo) pdt = L.flo;
        else if (pdt > L.fhi) pdt = L.fhi;
        jtau = pdt;
      }
    }
    nc = world_qacc(l, s, st, jtau, P, bqacc, jqacc);
    if (a.mode != 0) integrate_lane(L, st, bqacc, jqacc, a.guard != 0);
  }
  if (!wvalid) return;
  float* oa = a.qacc + (long)w * kNV;
  if (l == 1) {
#pragma unroll
    for (int k = 0; k < 6; ++k) oa[k] = bqacc[k];
    a.ncon[w] = nc;
  }
  if (L.hinge) oa[L.b + 4] = jqacc;
  if (a.mode != 0) {
    float* oq = a.qp + (long)w * kNQ;
    float* ov = a.qv + (long)w * kNV;
    if (l == 1) {
#pragma unroll
      for (int k = 0; k < 7; ++k) oq[k] = st.bq[k];
#pragma unroll
      for (int k = 0; k < 6; ++k) ov[k] = st.bqd[k];
    }
    if (L.hinge) { oq[L.b + 5] = st.jq; ov[L.b + 4] = st.jqd; }
  }
}

// ====================================================================== policy kernels
struct PolicyArgs {
  int ldx;                          // LDS row pitch (floats) of the activation tiles
  const float* qp; const float* qv; const float* pa; const unsigned* rng;
  int N, t, H;                      // t == H: bootstrap value only
  const float* mean; const float* var;
  PackedPolicy pp; PolicyShape shape;
  const float* act_noise;           // [H][N][29] or null (Philox)
  unsigned long long seed;
  float* O; float* A; float* LP; float* V; float* Vlast;
  const float* obs_in;              // probe mode: normalised observations [N][100] (skips obs/O)
  float* mu_out;                    // probe mode: [N][29] mean action
};

__global__ void __launch_bounds__(kPolicyThreads) __attribute__((amdgpu_waves_per_eu(4))) k_policy(PolicyArgs a) {
  // One activation buffer per tile, X[32][ld] (k-octet interleaved columns): the hidden layers
  // replace their input in place (mfma_layer_inplace), so two tiles fit in a CU's LDS at config 4's
  // widths. Columns past a phase's live data hold its staging: the tile's state at kPolicyStage..
  // and the normalisation constants at kPolicyConst.. (rows 0..9) during the observation, the
  // head's split-K partial tiles at ld - 256.. (policy_ldx sizes ld for all of them).
  extern __shared__ float smem[];
  const int ld = a.ldx;
  float* X = smem;
  const int tid = threadIdx.x;
  const int w0 = blockIdx.x * kTileWorlds;
  // ---- observation + frozen normalisation (reference: src/g1_env.cu:297-304)
  if (!a.obs_in) {
    // the tile's state first, with coalesced loads (qp, qv, pa of worlds w0.. are contiguous
    // blocks): world m's qpos, qvel and previous action at X[m][kPolicyStage + 0 | kNQ | kNQ + kNV]
    const int nw = a.N - w0 < kTileWorlds ? a.N - w0 : kTileWorlds;
    // the frozen statistics per feature i: mean, the divisor sqrt(var + 1e-8) and its RN
    // reciprocal (the quotient below is div_rn, the IEEE quotient), entry j of the 3 x kObs at
    // X[j / 32][kPolicyConst + j mod 32]
    auto cst = [&](int j) -> float& { return X[(j >> 5) * ld + kPolicyConst + (j & 31)]; };
    for (int i = tid; i < kObs; i += kPolicyThreads) {
      const float dv = sqrtf(a.var[i] + 1e-8f);
      cst(i) = a.mean[i];
      cst(kObs + i) = dv;
      cst(2 * kObs + i) = rcp_rn(dv);
    }
    for (int idx = tid; idx < kTileWorlds * (kNQ + kNV + kAct); idx += kPolicyThreads) {
      float v = 0.f;
      int m, c;
      if (idx < kTileWorlds * kNQ) {
        m = idx / kNQ; c = idx - m * kNQ;
        if (m < nw) v = a.qp[(long)w0 * kNQ + idx];
      } else if (idx < kTileWorlds * (kNQ + kNV)) {
        const int r = idx - kTileWorlds * kNQ;
        m = r / kNV; c = kNQ + r - m * kNV;
        if (m < nw) v = a.qv[(long)w0 * kNV + r];
      } else {
        const int r = idx - kTileWorlds * (kNQ + kNV);
        m = r / kAct; c = kNQ + kNV + r - m * kAct;
        if (m < nw) v = a.pa[(long)w0 * kAct + r];
      }
      X[m * ld + kPolicyStage + c] = v;
    }
    __syncthreads();
    // features go to columns kperm(i) < kPolicyStage: the staging is read, never overwritten
    for (int idx = tid; idx < kTileWorlds * kObs; idx += kPolicyThreads) {
      const int m = idx / kObs, i = idx - m * kObs;
      const int w = w0 + m;
      float z = 0.f;
      if (w < a.N) {
        const float* st = X + m * ld + kPolicyStage;
        const float o = obs_value(st, st + kNQ, st + kNQ + kNV, i);
        if (a.t < a.H) a.O[((long)a.t * a.N + w) * kObs + i] = o;
        z = div_rn_inf(o - cst(i), cst(kObs + i), cst(2 * kObs + i));
        if (z < -10.f) z = -10.f; else if (z > 10.f) z = 10.f;
      }
      X[m * ld + kperm(i)] = z;
    }
  } else {
    for (int idx = tid; idx < kTileWorlds * kObs; idx += kPolicyThreads) {
      const int m = idx / kObs, i = idx - m * kObs;
      const int w = w0 + m;
      X[m * ld + kperm(i)] = w < a.N ? a.obs_in[(long)w * kObs + i] : 0.f;
    }
  }
  // zero the first layer's K padding (observation index kObs .. K0 - 1; its weight rows are zero)
  for (int idx = tid; idx < kTileWorlds * (a.pp.K[0] - kObs); idx += kPolicyThreads) {
    const int m = idx / (a.pp.K[0] - kObs), i = kObs + idx % (a.pp.K[0] - kObs);
    X[m * ld + kperm(i)] = 0.f;
  }
  __syncthreads();
  // ---- hidden layers, each over its own input
  for (int ly = 0; ly < a.shape.nl; ++ly)
    mfma_layer_inplace(X, ld, a.pp.Wp + a.pp.woff[ly], a.pp.Wp + a.pp.boff[ly], a.pp.K[ly], a.pp.Np[ly],
                       a.shape.act);
  // ---- fused head [mu(29) | v | pad] into columns 0..31 (natural order)
  mfma_head_splitk(X, ld, ld - kPolicyWaves * 32, a.pp.Wp + a.pp.woff[a.shape.nl], a.pp.Wp + a.pp.boff[a.shape.nl],
                   a.pp.K[a.shape.nl]);
  __syncthreads();
  // ---- sampling + log-prob (reference: src/g1_env.cu:308-318): one thread per (world, action)
  // draws the noise and writes the action; each world's log-prob terms are then summed by one
  // thread in action order (the terms go to columns 32.. of the world's row)
  const float* head = X;
  float* lpt = X + 32;   // [32][ld]: log-prob terms
  const bool sample = !a.mu_out && a.t < a.H;
  if (sample) {
    // one thread per (world, action pair 2p, 2p + 1): both Box-Muller normals of one draw
    const float LOG2PI = 1.8378770664093453f;
    constexpr int kPairs = (kAct + 1) / 2;
    static_assert(kTileWorlds * kPairs <= kPolicyThreads, "one pass");
    const int m = tid / kPairs, pi = tid - m * kPairs;
    const int w = w0 + m;
    if (m < kTileWorlds && w < a.N) {
      const float* h = head + m * ld;
      const long ab = ((long)a.t * a.N + w) * kAct;
      float nz[2];
      if (a.act_noise) {
        nz[0] = a.act_noise[ab + 2 * pi];
        nz[1] = 2 * pi + 1 < kAct ? a.act_noise[ab + 2 * pi + 1] : 0.f;
      } else {
        rng_normal2(a.seed, w, a.rng[w], kStreamAction, pi, nz[0], nz[1]);
      }
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int i = 2 * pi + e;
        if (i < kAct) {
          const float ls = a.pp.log_std[i];
          a.A[ab + i] = h[i] + expf(ls) * nz[e];
          lpt[m * ld + i] = -0.5f * nz[e] * nz[e] - ls - 0.5f * LOG2PI;
        }
      }
    }
    __syncthreads();
  }
  if (tid < kTileWorlds) {
    const int w = w0 + tid;
    if (w < a.N) {
      const float* h = head + tid * ld;
      const float val = h[kAct];
      if (a.mu_out) {
        for (int i = 0; i < kAct; ++i) a.mu_out[(long)w * kAct + i] = h[i];
        a.V[w] = val;
      } else if (a.t == a.H) {
        a.Vlast[w] = val;
      } else {
        float lpsum = 0.f;
        for (int i = 0; i < kAct; ++i) lpsum += lpt[tid * ld + i];
        a.LP[(long)a.t * a.N + w] = lpsum;
        a.V[(long)a.t * a.N + w] = val;
      }
    }
  }
}

// Pack torch-order weights W0,b0,..,Wmu,bmu,Wv,bv,log_std into MFMA layout (k-pair major).
struct PackArgs {
  const float* W; float* Wp; PackedPolicy pp; PolicyShape shape; long total;
};
__global__ void k_pack(PackArgs a) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.total) return;
  // locate layer
  int ly = 0;
  while (ly < a.shape.nl && idx >= a.pp.woff[ly + 1]) ++ly;
  const long base = a.pp.woff[ly];
  const long rel = idx - base;
  const int K = a.pp.K[ly], Np = a.pp.Np[ly];
  const long wsize = (long)K * Np;
  // source offsets in torch order
  long src = 0;
  int in = kObs;
  for (int q = 0; q < ly; ++q) { src += (long)a.shape.hid[q] * in + a.shape.hid[q]; in = a.shape.hid[q]; }
  const int Kin = in;
  if (rel < wsize) {
    // k-octet-major: rel = ((o * Np + n) * 2 + khalf) * 4 + j holds W[n][8o + 2j + khalf]
    const int j = (int)(rel & 3), khalf = (int)((rel >> 2) & 1);
    const long r8 = rel >> 3;
    const int n = (int)(r8 % Np), o = (int)(r8 / Np);
    const int k = 8 * o + 2 * j + khalf;
    float v = 0.f;
    if (ly < a.shape.nl) {
      if (n < a.shape.hid[ly] && k < Kin) v = a.W[src + (long)n * Kin + k];
    } else if (k < Kin) {
      if (n < kAct) v = a.W[src + (long)n * Kin + k];                       // Wmu
      else if (n == kAct) v = a.W[src + (long)kAct * Kin + kAct + k];        // Wv
    }
    a.Wp[idx] = v;
  } else {
    const int n = (int)(rel - wsize);
    float v = 0.f;
    if (ly < a.shape.nl) {
      if (n < a.shape.hid[ly]) v = a.W[src + (long)a.shape.hid[ly] * Kin + n];
    } else {
      if (n < kAct) v = a.W[src + (long)kAct * Kin + n];                          // bmu
      else if (n == kAct) v = a.W[src + (long)kAct * Kin + kAct + Kin];            // bv
    }
    a.Wp[idx] = v;
  }
}

// ---- reset (reference: src/g1_env.cu:97-111) and observation export
__global__ void k_reset(float* qp, float* qv, float* pa, int* steps, unsigned* rng, int N, float noise,
                        const float* inj, unsigned long long seed) {
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= N) return;
  float* gq = qp + (long)w * kNQ;
  for (int i = 0; i < kNQ; ++i) gq[i] = MF::qpos_stand[i];
  for (int i = 0; i < kAct; ++i) {
    const float u = inj ? inj[(long)w * kAct + i] : rng_pm1(seed, w, rng[w], kStreamInit, i);
    gq[act_qadr[i]] += noise * u;
  }
  for (int i = 0; i < kNV; ++i) qv[(long)w * kNV + i] = 0.f;
  for (int i = 0; i < kAct; ++i) pa[(long)w * kAct + i] = 0.f;
  steps[w] = 0;
  rng[w] += 1;
}

__global__ void k_obs(const float* qp, const float* qv, const float* pa, int N, float* obs) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)N * kObs) return;
  const int w = (int)(idx / kObs), i = (int)(idx % kObs);
  obs[idx] = obs_value(qp + (long)w * kNQ, qv + (long)w * kNV, pa + (long)w * kAct, i);
}

__global__ void k_philox(const unsigned* in, unsigned* out, int n, unsigned k0, unsigned k1) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  U4 r = philox4x32_10(U4{in[4 * i], in[4 * i + 1], in[4 * i + 2], in[4 * i + 3]}, k0, k1);
  out[4 * i] = r.x; out[4 * i + 1] = r.y; out[4 * i + 2] = r.z; out[4 * i + 3] = r.w;
}

// rcp_rn / div_rn of the physics kernel on caller-given operands (parity probe)
__global__ void k_divide(const float* a, const float* b, float* rcp, float* quot, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float y = rcp_rn(b[i]);
  rcp[i] = y;
  quot[i] = div_rn(a[i], b[i], y);
}

// sqrt_rn_pos of the physics kernel (the Cholesky pivots) on caller-given arguments (parity probe)
__global__ void k_sqrt(const float* x, float* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = sqrt_rn_pos(x[i]);
}

// sincos_small_rn of the physics kernel on caller-given arguments (parity probe)
__global__ void k_sincos(const float* x, float* sn, float* cs, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s, c;
  sincos_small_rn(x[i], s, c);
  sn[i] = s;
  cs[i] = c;
}

// sincos_hinge_rn of the physics kernel (the FK's hinge half-angles) on caller-given arguments
__global__ void k_sincos_hinge(const float* x, float* sn, float* cs, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s, c;
  sincos_hinge_rn(x[i], s, c);
  sn[i] = s;
  cs[i] = c;
}

// ====================================================================== host side
struct EnvState {
  int N, S, pgs;
  unsigned long long seed;
  float mu;
  PolicyShape shape;
  float *qp, *qv, *pa;
  int* steps;
  unsigned* rng;
  float *dact, *zero_act, *bench_r, *bench_d;
  float* dout;            // host-step outputs on the device: [obs N x 100 | reward N | done N]
  float *h_act, *h_out;   // pinned host staging of the host-step path: actions in; obs, reward, done, queue error out
  hipEvent_t step_ev[kStepChunks + 1];   // host-step output copies done: observation chunks, reward/done
  float* Wp;
  long Wp_cap;
  unsigned long long* ncon_hist;
  int hist_on;
  // physics work queue (k_physics): per-pair item flags, claim counters, split-step accumulators
  unsigned* qflags;
  unsigned* qctr;
  int* qerr;
  float *qacc_e, *qacc_vx;
  unsigned qdone;   // value of every pair flag after the launches enqueued so far
  int qpar;         // counter row of the next launch
  int pgrid;        // persistent grid: resident blocks of k_physics, a multiple of kQueues
  int xlocal;       // blocks land on XCD blockIdx % kXcds (measured at creation)
  int fences;       // 1: hand over state with agent-scope fences even where xlocal holds
  // one-launch rollout (k_rollout): policy tiles' flags, their completed-step count, packed weights
  int fused;        // 1: g1_rollout runs k_rollout when the policy shape allows it
  unsigned* tflags;
  unsigned* tcount;
  unsigned long long* tperm;   // per tile: the pairing of its worlds in the current step
  unsigned char* cflag;        // per world: contacts at the last substep of its last control step
  unsigned tdone;
  float* Wt;
  long Wt_cap;
  float* scr;       // wide one-launch policy: per block two activation buffers (WideLayout::maxT * 256 floats each)
  long scr_cap;
  int* h_qerr;      // pinned copy of qerr, refreshed asynchronously after every rollout
  // per-launch HIP events of the rollout's physics / policy kernels (null stream)
  int prof_on;
  std::vector<hipEvent_t> ev_phys, ev_pol;
  size_t n_phys, n_pol;
  long dev_bytes;   // device memory held (g1_env_device_bytes)
};

// Device allocations of an env, counted in dev_bytes.
template <class T>
static void dev_alloc(EnvState* E, T** p, size_t bytes) {
  HIPCHECK(hipMalloc((void**)p, bytes));
  E->dev_bytes += (long)bytes;
}
static void dev_free(EnvState* E, void* p, size_t bytes) {
  HIPCHECK(hipFree(p));
  E->dev_bytes -= (long)bytes;
}

static void prof_mark(std::vector<hipEvent_t>& v, size_t& n) {
  if (n == v.size()) {
    hipEvent_t e;
    HIPCHECK(hipEventCreate(&e));
    v.push_back(e);
  }
  HIPCHECK(hipEventRecord(v[n++], 0));
}

static PackedPolicy make_packed(const PolicyShape& sh, float* Wp, const float* W, long* total) {
  PackedPolicy pp{};
  pp.Wp = Wp;
  long off = 0;
  int in = kObs;
  for (int ly = 0; ly <= sh.nl; ++ly) {
    const int out = ly < sh.nl ? sh.hid[ly] : 32;
    pp.K[ly] = (in + 7) & ~7;
    pp.Np[ly] = (out + 31) & ~31;
    pp.woff[ly] = off;   // a multiple of 4 floats: every term below is (float4 loads)
    off += (long)pp.K[ly] * pp.Np[ly];
    pp.boff[ly] = off;
    off += pp.Np[ly];
    if (ly < sh.nl) in = sh.hid[ly];
  }
  // pack-kernel layer search uses woff[nl+1] as the end sentinel
  if (sh.nl + 1 <= kMaxLayers) pp.woff[sh.nl + 1] = off;
  *total = off;
  long nparam = 0;
  in = kObs;
  for (int ly = 0; ly < sh.nl; ++ly) { nparam += (long)sh.hid[ly] * in + sh.hid[ly]; in = sh.hid[ly]; }
  nparam += (long)kAct * in + kAct + in + 1;
  pp.log_std = W ? W + nparam : nullptr;
  return pp;
}

static long policy_param_count(const PolicyShape& sh) {
  long n = 0;
  int in = kObs;
  for (int ly = 0; ly < sh.nl; ++ly) { n += (long)sh.hid[ly] * in + sh.hid[ly]; in = sh.hid[ly]; }
  return n + (long)kAct * in + kAct + in + 1 + kAct;
}

static int max_width(const PolicyShape& sh) {
  int m = kObs;
  for (int ly = 0; ly < sh.nl; ++ly) m = sh.hid[ly] > m ? sh.hid[ly] : m;
  return m;
}

// Packs W into dst (capacity dst_cap floats, no allocation) or, with dst null, into the env's own
// buffer, grown with hipMalloc as the policy shape requires.
static void pack_policy(EnvState* E, const float* W, PackedPolicy* out, float* dst = nullptr, long dst_cap = 0) {
  long total = 0;
  PackedPolicy pp = make_packed(E->shape, nullptr, W, &total);
  float* Wp = dst;
  if (!Wp) {
    if (total > E->Wp_cap) {
      if (E->Wp) dev_free(E, E->Wp, E->Wp_cap * sizeof(float));
      dev_alloc(E, &E->Wp, total * sizeof(float));
      E->Wp_cap = total;
    }
    Wp = E->Wp;
  } else if (total > dst_cap) {
    fail("pack_policy: packed policy larger than its buffer");
  }
  pp = make_packed(E->shape, Wp, W, &total);
  PackArgs pa{W, Wp, pp, E->shape, total};
  hipLaunchKernelGGL(k_pack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, 0, pa);
  HIPCHECK(hipGetLastError());
  *out = pp;
}

// activation tile pitch: the widest of (every layer's width, the head's input plus its split-K
// partial tiles, the observation staging) rounded up to the 32-column tiles, + 4 floats (keeps rows
// off the same LDS banks; a multiple of 4 for the 16-byte operand reads)
static int policy_ldx(const PolicyShape& sh) {
  int m = max_width(sh);
  const int khead = (sh.hid[sh.nl - 1] + 7) / 8 * 8;   // the head's K (make_packed pads to 8)
  m = khead + kPolicyWaves * 32 > m ? khead + kPolicyWaves * 32 : m;
  m = kPolicyConst + 32 > m ? kPolicyConst + 32 : m;
  return (m + 31) / 32 * 32 + 4;
}
static size_t policy_smem(const PolicyShape& sh) { return (size_t)kTileWorlds * policy_ldx(sh) * sizeof(float); }

static void launch_policy_kernel(const PolicyArgs& a, int N, const PolicyShape& sh) {
  const size_t smem = policy_smem(sh);
  static size_t granted = 0;
  if (smem > granted) {
    HIPCHECK(hipFuncSetAttribute((const void*)k_policy, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    granted = smem;
  }
  hipLaunchKernelGGL(k_policy, dim3((N + kTileWorlds - 1) / kTileWorlds), dim3(kPolicyThreads), smem, 0, a);
  HIPCHECK(hipGetLastError());
}

static void launch_policy(EnvState* E, const PackedPolicy& pp, int t, int H, const float* mean, const float* var,
                          const float* act_noise, float* O, float* A, float* LP, float* V, float* Vlast) {
  PolicyArgs a{};
  a.qp = E->qp; a.qv = E->qv; a.pa = E->pa; a.rng = E->rng;
  a.N = E->N; a.t = t; a.H = H; a.mean = mean; a.var = var; a.pp = pp; a.shape = E->shape;
  a.act_noise = act_noise; a.seed = E->seed;
  a.O = O; a.A = A; a.LP = LP; a.V = V; a.Vlast = Vlast;
  a.ldx = policy_ldx(E->shape);
  launch_policy_kernel(a, E->N, E->shape);
}

static PhysArgs phys_args(EnvState* E) {
  PhysArgs a{};
  a.qp = E->qp; a.qv = E->qv; a.pa = E->pa; a.steps = E->steps; a.rng = E->rng;
  a.N = E->N; a.S = E->S; a.pgs = E->pgs; a.K = 1; a.mu = E->mu; a.seed = E->seed;
  a.ncon_hist = E->hist_on ? E->ncon_hist : nullptr;
  a.flags = E->qflags; a.qctr = E->qctr; a.acc = E->qacc_e; a.vxs = E->qacc_vx; a.qerr = E->qerr;
  return a;
}

// Substep chunks of a control step, the work items of one pair. Large items amortise the hand-over
// of a pair's state between waves; small last items shorten the launch's tail, which matters when
// each wave holds little work. Measured at S = 10 (same-box A/B of the physics launch):
// * 2 pairs per wave (config 3, N = 8192): 3,3,2,2 0.434 ms; 4,3,3 0.440; 3,3,2,1,1 0.442;
//   2,2,2,2,1,1 0.444; 4,4,2 0.446; 4,3,2,1 0.448; 2 x 5 0.437; 3,3,3,1 0.457; 5,5 0.466.
// * 32 pairs per wave (config 4, N = 131072): 6,4 5.81 ms; 5,5 5.83; 10 5.83; 4,3,3 5.86;
//   2 x 5 5.98; 2,2,2,2,1,1 6.02.
// In the one-launch rollout (one_launch) the policy items keep the waves busy across control
// steps, and a whole control step per item does best (config 3, ms per rollout, every step cut the
// same way): 10 12.82; 6,4 12.87-12.91; 5,5 12.88; 7,3 12.91; 4,3,3 13.01; 2,2,2,2,2 13.56.
static void chunk_schedule(PhysArgs& a, int pgrid, bool one_launch = false) {
  const int S = a.S;
  // kind 0: one item; 1: 60% then the rest; 2: three-substep items (longer for S > 46, within
  // kMaxChunks) while more than four substeps remain, then two, a single one last
  auto build = [&](int kind, int* cst) {
    int n = 0, s0 = 0;
    auto add = [&](int len) { cst[n++] = s0; s0 += len; };
    if (kind == 0) {
      add(S);
    } else if (kind == 1) {
      const int first = (3 * S + 4) / 5;
      add(first);
      if (S > first) add(S - first);
    } else {
      const int big = std::max(3, (S - 4 + kMaxChunks - 3) / (kMaxChunks - 2));
      while (S - s0 > 4) add(std::min(big, S - s0 - 2));
      while (s0 < S) add(S - s0 >= 2 ? 2 : 1);
    }
    cst[n] = S;
    if (n < 1 || n > kMaxChunks || s0 != S) fail("physics launch: bad substep chunk schedule");
    for (int c = 0; c < n; ++c)
      if (cst[c + 1] <= cst[c]) fail("physics launch: bad substep chunk schedule");
    return n;
  };
  const double work_per_wave = (double)((a.N + 1) / 2) * a.K / pgrid;   // pair-control-steps
  const bool big = work_per_wave >= 8.0;
  a.nch = build(one_launch && big ? 0 : (big ? 1 : 2), a.cst);
  // the one-launch rollout ends its last control step in two items, which shortens the launch's
  // drain (config 3, ms per rollout, same-box A/B: last step as 6,4 12.80; 3,3,2,2 12.80;
  // 2,2,2,2,1,1 12.83; ten single substeps 12.86; one item 12.84-12.87)
  a.nchl = build(big ? 1 : 2, a.cstl);
}

// Enqueue one physics launch on the null stream; the queue state (flag base, counter row) advances
// on the host in launch order, which is the stream's execution order.
static void launch_physics(EnvState* E, PhysArgs& a) {
  if (a.K <= 0) fail("physics launch: K must be positive");
  chunk_schedule(a, E->pgrid);
  const long per_pair = (long)(a.K - 1) * a.nch + a.nchl;
  if (per_pair > (1L << 30)) fail("physics launch: too many work items per pair");
  a.fbase = E->qdone;
  a.qpar = E->qpar;
  a.xlocal = E->xlocal && !E->fences;
  hipLaunchKernelGGL(k_physics, dim3((unsigned)E->pgrid), dim3(kPhysThreads), 0, 0, a);
  HIPCHECK(hipGetLastError());
  E->qdone += (unsigned)per_pair;
  E->qpar ^= 1;
}

// The work queue's error word (nonzero: a physics launch saw a dependency wait exceed its bound,
// or a block off its queue's XCD; results are then undefined): print and exit, as HIP errors do.
static void check_queue_error(int err) {
  if (err == 1) fail("physics work queue: a dependency wait exceeded its bound");
  if (err) fail("physics work queue: a block ran outside the XCD its queue was placed on");
}

static void check_queue(EnvState* E) {
  int err = 0;
  HIPCHECK(hipMemcpy(&err, E->qerr, sizeof(int), hipMemcpyDeviceToHost));
  check_queue_error(err);
}

// The asynchronous entry points (g1_rollout*) end with a copy of the error word into pinned host
// memory; every later entry reads that copy without synchronising, so an error stops the caller at
// its next call into the library once the copy has landed (and at the latest in g1_env_destroy or
// at the next synchronising call, which read the device word itself).
static void poll_queue_error(EnvState* E) {
  check_queue_error(*(volatile int*)E->h_qerr);
}

// The one-launch rollout runs policies of two hidden layers of at most 256 units each on the
// register-resident tile (policy_tile, at 256-256 with zero padding) and every other accepted shape
// (1..3 hidden layers of at most 512 units) on the wide tile (policy_tile_wide, activations staged
// in global memory). The split form (policy and physics launches per control step) remains for
// g1_env_set_fused(h, 0) and for g1_rollout_noalloc with a wide shape (the wide tile's activation
// buffers are allocated by the library).
static bool narrow_shape(const PolicyShape& sh) {
  return sh.nl == 2 && sh.hid[0] <= kTileMaxHidden && sh.hid[1] <= kTileMaxHidden;
}
static bool fused_shape(const PolicyShape& sh, bool noalloc) {
  return narrow_shape(sh) || !noalloc;
}

static int tiles_per_queue(int N) {
  const int npairs = (N + 1) / 2;
  const int nq = (npairs + kQueues - 1) / kQueues;
  return (nq + kTilePairs - 1) / kTilePairs;
}

// The whole rollout as one k_rollout launch on the null stream; wp (capacity wp_cap floats) takes
// the tile-packed weights instead of the env's own buffer.
static void rollout_fused(EnvState* E, int H, const float* W, const float* mean, const float* var, float* O, float* A,
                          float* LP, float* V, float* R, float* D, float* Vlast, const float* act_noise,
                          const float* reset_noise, float* wp, long wp_cap) {
  const bool wide = !narrow_shape(E->shape);
  const TileLayout tl = tile_layout(E->shape.act);
  const WideLayout wl = wide_layout(E->shape.nl, E->shape.hid, E->shape.act);
  const long total = wide ? wl.total : tl.total;
  float* Wt = wp;
  if (!Wt) {
    if (total > E->Wt_cap) {
      if (E->Wt) dev_free(E, E->Wt, E->Wt_cap * sizeof(float));
      dev_alloc(E, &E->Wt, total * sizeof(float));
      E->Wt_cap = total;
    }
    Wt = E->Wt;
  } else if (total > wp_cap) {
    fail("rollout: tile-packed policy larger than its buffer");
  }
  float* scr = nullptr;
  if (wide) {
    if (wp) fail("rollout: the wide one-launch policy needs the library's activation buffers");
    const long need = (long)E->pgrid * 2 * wl.maxT * 256;
    if (need > E->scr_cap) {
      if (E->scr) dev_free(E, E->scr, E->scr_cap * sizeof(float));
      dev_alloc(E, &E->scr, need * sizeof(float));
      E->scr_cap = need;
    }
    scr = E->scr;
    WidePackArgs pk{W, mean, var, Wt, wl, {0, 0, 0, 0}};
    for (int i = 0; i < E->shape.nl; ++i) pk.hid[i] = E->shape.hid[i];
    hipLaunchKernelGGL(k_pack_wide, dim3((unsigned)((wl.total + 255) / 256)), dim3(256), 0, 0, pk);
  } else {
    TilePackArgs pk{W, mean, var, Wt, tl, E->shape.hid[0], E->shape.hid[1]};
    hipLaunchKernelGGL(k_pack_tiles, dim3((unsigned)((tl.total + 255) / 256)), dim3(256), 0, 0, pk);
  }
  HIPCHECK(hipGetLastError());
  RolloutArgs ra{};
  ra.ph = phys_args(E);
  PhysArgs& a = ra.ph;
  a.K = H; a.act = A; a.t0 = 0; a.astep = 1; a.rstep = 1; a.R = R; a.D = D; a.reset_noise = reset_noise;
  chunk_schedule(a, E->pgrid, true);
  a.fbase = E->qdone;
  a.qpar = E->qpar;
  a.xlocal = E->xlocal && !E->fences;
  ra.po = TileArgs{Wt, tl, act_noise, O, A, LP, V, Vlast, H, wide ? 1 : 0, wl, scr};
  ra.tflags = E->tflags;
  ra.tbase = E->tdone;
  ra.tcount = E->tcount;
  ra.tperm = E->tperm;
  a.cflag = E->cflag;
  const bool prof = E->prof_on != 0 && !wp;
  if (prof) prof_mark(E->ev_phys, E->n_phys);
  launch_rollout_kernel(ra, E->pgrid);
  HIPCHECK(hipGetLastError());
  if (prof) prof_mark(E->ev_phys, E->n_phys);
  E->qdone += H > 0 ? (unsigned)((H - 1) * a.nch + a.nchl) : 0u;
  E->tdone += (unsigned)H + 1u;
  E->qpar ^= 1;
  HIPCHECK(hipMemcpyAsync(E->h_qerr, E->qerr, sizeof(int), hipMemcpyDeviceToHost, 0));
}

static void rollout_impl(EnvState* E, int H, const float* W, const float* mean, const float* var, float* O, float* A,
                         float* LP, float* V, float* R, float* D, float* Vlast, const float* act_noise,
                         const float* reset_noise, float* wp = nullptr, long wp_cap = 0) {
  poll_queue_error(E);
  if (H < 0) H = 0;   // no control step; the bootstrap value is still computed (as the reference's k_rollout)
  if (E->fused && fused_shape(E->shape, wp != nullptr)) {
    rollout_fused(E, H, W, mean, var, O, A, LP, V, R, D, Vlast, act_noise, reset_noise, wp, wp_cap);
    return;
  }
  PackedPolicy pp;
  pack_policy(E, W, &pp, wp, wp_cap);
  PhysArgs pa = phys_args(E);
  pa.act = A; pa.astep = 1; pa.rstep = 1; pa.R = R; pa.D = D; pa.reset_noise = reset_noise;
  const bool prof = E->prof_on != 0 && !wp;
  for (int t = 0; t < H; ++t) {
    if (prof) prof_mark(E->ev_pol, E->n_pol);
    launch_policy(E, pp, t, H, mean, var, act_noise, O, A, LP, V, Vlast);
    if (prof) { prof_mark(E->ev_pol, E->n_pol); prof_mark(E->ev_phys, E->n_phys); }
    pa.t0 = t;
    launch_physics(E, pa);
    if (prof) prof_mark(E->ev_phys, E->n_phys);
  }
  if (prof) prof_mark(E->ev_pol, E->n_pol);
  launch_policy(E, pp, H, H, mean, var, act_noise, O, A, LP, V, Vlast);
  if (prof) prof_mark(E->ev_pol, E->n_pol);
  HIPCHECK(hipMemcpyAsync(E->h_qerr, E->qerr, sizeof(int), hipMemcpyDeviceToHost, 0));
}

// ---- packed policy weights of g1_rollout_noalloc: a file-scope device array, so the entry point
// allocates nothing. The widest shape g1_env_set_policy accepts (three hidden layers of 512) packs
// into 595,488 floats; the array holds 640 Ki floats (2.5 MiB) on every GPU the library runs on,
// until the process ends. Host code never names the array in a launch: it uses the device address
// hipGetSymbolAddress returns, once per device, with that device current (kept in scratch_addr).
constexpr long kScratchFloats = 640L * 1024L;
static __device__ __align__(256) float scratch[kScratchFloats];
constexpr int kMaxDevices = 64;
static float* scratch_addr[kMaxDevices];

static void scratch_setup() {
  int dev = 0;
  HIPCHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) fail("scratch_setup: device index beyond the library's table");
  if (scratch_addr[dev]) return;
  void* p = nullptr;
  HIPCHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  scratch_addr[dev] = (float*)p;
}

extern "C" {

int g1_env_obs_dim(void) { return kObs; }
int g1_env_act_dim(void) { return kAct; }

void* g1_env_create(int N, int substeps, int pgs_iters, unsigned long seed) {
  if (N <= 0 || substeps <= 0 || pgs_iters < 0) fail("g1_env_create: invalid N/substeps/pgs_iters");
  scratch_setup();
  EnvState* E = new EnvState();
  E->N = N; E->S = substeps; E->pgs = pgs_iters; E->seed = seed; E->mu = MF::foot_mu;
  E->shape = PolicyShape{2, {256, 256, 0, 0}, 0};
  dev_alloc(E, &E->qp, (size_t)N * kNQ * 4);
  dev_alloc(E, &E->qv, (size_t)N * kNV * 4);
  dev_alloc(E, &E->pa, (size_t)N * kAct * 4);
  dev_alloc(E, &E->steps, (size_t)N * 4);
  dev_alloc(E, &E->rng, (size_t)N * 4);
  dev_alloc(E, &E->dact, (size_t)N * kAct * 4);
  dev_alloc(E, &E->zero_act, (size_t)N * kAct * 4);
  dev_alloc(E, &E->bench_r, (size_t)N * 4);
  dev_alloc(E, &E->bench_d, (size_t)N * 4);
  dev_alloc(E, &E->ncon_hist, 9 * sizeof(unsigned long long));
  const int npairs = (N + 1) / 2;
  dev_alloc(E, &E->qflags, (size_t)npairs * sizeof(unsigned));
  dev_alloc(E, &E->qctr, 2 * kQueues * sizeof(unsigned));
  dev_alloc(E, &E->qerr, sizeof(int));
  dev_alloc(E, &E->qacc_e, (size_t)N * kGroup * 4);
  dev_alloc(E, &E->qacc_vx, (size_t)N * 4);
  HIPCHECK(hipMemset(E->qflags, 0, (size_t)npairs * sizeof(unsigned)));
  HIPCHECK(hipMemset(E->qctr, 0, 2 * kQueues * sizeof(unsigned)));
  HIPCHECK(hipMemset(E->qerr, 0, sizeof(int)));
  E->qdone = 0; E->qpar = 0;
  dev_alloc(E, &E->tflags, (size_t)kQueues * tiles_per_queue(N) * sizeof(unsigned));
  HIPCHECK(hipMemset(E->tflags, 0, (size_t)kQueues * tiles_per_queue(N) * sizeof(unsigned)));
  dev_alloc(E, &E->tcount, (size_t)kQueues * tiles_per_queue(N) * sizeof(unsigned));
  HIPCHECK(hipMemset(E->tcount, 0, (size_t)kQueues * tiles_per_queue(N) * sizeof(unsigned)));
  dev_alloc(E, &E->tperm, (size_t)kQueues * tiles_per_queue(N) * sizeof(unsigned long long));   // set by each launch
  dev_alloc(E, &E->cflag, (size_t)N);
  HIPCHECK(hipMemset(E->cflag, 0, (size_t)N));
  E->tdone = 0;
  E->fused = 1;
  {
    // persistent grid: every resident block of k_physics, in whole rounds of the kQueues queues,
    // and no more blocks than there are pairs (rounded up to the queues)
    int dev = 0, cus = 0, per_cu = 0;
    HIPCHECK(hipGetDevice(&dev));
    HIPCHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    HIPCHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k_physics, kPhysThreads, 0));
    int cap = (cus * (per_cu > 0 ? per_cu : 1)) / kQueues * kQueues;
    if (cap < kQueues) cap = kQueues;
    const int need = (npairs + kQueues - 1) / kQueues * kQueues;
    E->pgrid = need < cap ? need : cap;
    // placement of the blocks on the XCDs: round-robin lets each queue hand over state in one L2
    int* dx = nullptr;
    HIPCHECK(hipMalloc(&dx, (size_t)E->pgrid * sizeof(int)));
    hipLaunchKernelGGL(k_xcc, dim3((unsigned)E->pgrid), dim3(kPhysThreads), 0, 0, dx);
    HIPCHECK(hipGetLastError());
    std::vector<int> hx(E->pgrid);
    HIPCHECK(hipMemcpy(hx.data(), dx, (size_t)E->pgrid * sizeof(int), hipMemcpyDeviceToHost));
    HIPCHECK(hipFree(dx));
    E->xlocal = 1;
    for (int b = 0; b < E->pgrid; ++b)
      if (hx[b] != b % kXcds) E->xlocal = 0;
  }
  dev_alloc(E, &E->dout, (size_t)N * (kObs + 2) * 4);
  HIPCHECK(hipHostMalloc((void**)&E->h_act, (size_t)N * kAct * 4, hipHostMallocDefault));
  HIPCHECK(hipHostMalloc((void**)&E->h_out, ((size_t)N * (kObs + 2) + 1) * 4, hipHostMallocDefault));
  HIPCHECK(hipHostMalloc((void**)&E->h_qerr, sizeof(int), hipHostMallocDefault));
  *E->h_qerr = 0;
  for (hipEvent_t& e : E->step_ev) HIPCHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  HIPCHECK(hipMemset(E->zero_act, 0, (size_t)N * kAct * 4));
  HIPCHECK(hipMemset(E->rng, 0, (size_t)N * 4));
  HIPCHECK(hipMemset(E->ncon_hist, 0, 9 * sizeof(unsigned long long)));
  // defined start state (the reference leaves it undefined until reset)
  hipLaunchKernelGGL(k_reset, dim3((N + 255) / 256), dim3(256), 0, 0, E->qp, E->qv, E->pa, E->steps, E->rng, N, 0.f,
                     (const float*)nullptr, E->seed);
  HIPCHECK(hipGetLastError());
  HIPCHECK(hipMemset(E->rng, 0, (size_t)N * 4));
  HIPCHECK(hipDeviceSynchronize());
  return E;
}

void g1_env_destroy(void* h) {
  EnvState* E = (EnvState*)h;
  if (!E) return;
  HIPCHECK(hipDeviceSynchronize());
  check_queue(E);
  void* bufs[] = {E->qp,       E->qv,      E->pa,        E->steps,   E->rng,  E->dact,
                  E->zero_act, E->bench_r, E->bench_d,   E->ncon_hist, E->Wp,  E->dout,
                  E->qflags,   E->qctr,    E->qerr,      E->qacc_e,  E->qacc_vx, E->tflags, E->tcount, E->tperm,
                  E->cflag,    E->Wt,      E->scr};
  for (void* b : bufs)
    if (b) HIPCHECK(hipFree(b));
  if (E->h_act) HIPCHECK(hipHostFree(E->h_act));
  if (E->h_out) HIPCHECK(hipHostFree(E->h_out));
  if (E->h_qerr) HIPCHECK(hipHostFree(E->h_qerr));
  for (auto e : E->ev_phys) (void)hipEventDestroy(e);
  for (hipEvent_t e : E->step_ev) (void)hipEventDestroy(e);
  for (auto e : E->ev_pol) (void)hipEventDestroy(e);
  delete E;
}

void g1_env_reset(void* h, float* obs_out) {
  EnvState* E = (EnvState*)h;
  poll_queue_error(E);
  const int N = E->N;
  hipLaunchKernelGGL(k_reset, dim3((N + 255) / 256), dim3(256), 0, 0, E->qp, E->qv, E->pa, E->steps, E->rng, N, 0.02f,
                     (const float*)nullptr, E->seed);
  HIPCHECK(hipGetLastError());
  hipLaunchKernelGGL(k_obs, dim3((unsigned)(((long)N * kObs + 255) / 256)), dim3(256), 0, 0, E->qp, E->qv, E->pa, N,
                     E->dout);
  HIPCHECK(hipGetLastError());
  HIPCHECK(hipMemcpyAsync(E->h_out, E->dout, (size_t)N * kObs * 4, hipMemcpyDeviceToHost, 0));
  HIPCHECK(hipStreamSynchronize(0));
  std::memcpy(obs_out, E->h_out, (size_t)N * kObs * 4);
}

// Host-step path (reference: src/g1_env.cu:245-268,431-441): actions staged through pinned memory,
// one launch that also writes the observation, one device-to-host copy of [obs | reward | done].
void g1_env_step(void* h, const float* act, float* obs, float* rew, float* done) {
  EnvState* E = (EnvState*)h;
  poll_queue_error(E);
  const int N = E->N;
  // The caller's arrays are pageable: they pass through the pinned staging in chunks of worlds,
  // so the host copy of one chunk overlaps the DMA of another.
  const size_t per = ((size_t)N + kStepChunks - 1) / kStepChunks;
  for (int c = 0; c < kStepChunks; ++c) {
    const size_t w0 = c * per, w1 = w0 + per < (size_t)N ? w0 + per : (size_t)N;
    if (w0 >= w1) break;
    std::memcpy(E->h_act + w0 * kAct, act + w0 * kAct, (w1 - w0) * kAct * 4);
    HIPCHECK(hipMemcpyAsync(E->dact + w0 * kAct, E->h_act + w0 * kAct, (w1 - w0) * kAct * 4, hipMemcpyHostToDevice, 0));
  }
  PhysArgs pa = phys_args(E);
  pa.act = E->dact; pa.t0 = 0; pa.astep = 0; pa.rstep = 0;
  pa.obs = E->dout; pa.R = E->dout + (size_t)N * kObs; pa.D = E->dout + (size_t)N * (kObs + 1);
  launch_physics(E, pa);
  for (int c = 0; c < kStepChunks; ++c) {
    const size_t w0 = c * per, w1 = w0 + per < (size_t)N ? w0 + per : (size_t)N;
    if (w0 < w1)
      HIPCHECK(hipMemcpyAsync(E->h_out + w0 * kObs, E->dout + w0 * kObs, (w1 - w0) * kObs * 4, hipMemcpyDeviceToHost, 0));
    HIPCHECK(hipEventRecord(E->step_ev[c], 0));
  }
  HIPCHECK(hipMemcpyAsync(E->h_out + (size_t)N * kObs, E->dout + (size_t)N * kObs, (size_t)N * 2 * 4,
                          hipMemcpyDeviceToHost, 0));
  HIPCHECK(hipMemcpyAsync(E->h_out + (size_t)N * (kObs + 2), E->qerr, sizeof(int), hipMemcpyDeviceToHost, 0));
  HIPCHECK(hipEventRecord(E->step_ev[kStepChunks], 0));
  for (int c = 0; c < kStepChunks; ++c) {
    HIPCHECK(hipEventSynchronize(E->step_ev[c]));
    const size_t w0 = c * per, w1 = w0 + per < (size_t)N ? w0 + per : (size_t)N;
    if (w0 < w1) std::memcpy(obs + w0 * kObs, E->h_out + w0 * kObs, (w1 - w0) * kObs * 4);
  }
  HIPCHECK(hipEventSynchronize(E->step_ev[kStepChunks]));
  int err;
  std::memcpy(&err, E->h_out + (size_t)N * (kObs + 2), sizeof(int));
  check_queue_error(err);
  std::memcpy(rew, E->h_out + (size_t)N * kObs, (size_t)N * 4);
  std::memcpy(done, E->h_out + (size_t)N * (kObs + 1), (size_t)N * 4);
}

void g1_rollout(void* h, int H, const float* W, const float* mean, const float* var, float* O, float* A, float* LP,
                float* V, float* R, float* D, float* Vlast) {
  rollout_impl((EnvState*)h, H, W, mean, var, O, A, LP, V, R, D, Vlast, nullptr, nullptr);
}

void g1_rollout_ex(void* h, int H, const float* W, const float* mean, const float* var, float* O, float* A, float* LP,
                   float* V, float* R, float* D, float* Vlast, const float* act_noise, const float* reset_noise) {
  rollout_impl((EnvState*)h, H, W, mean, var, O, A, LP, V, R, D, Vlast, act_noise, reset_noise);
}

int g1_rollout_noalloc(void* h, int H, const float* W, const float* mean, const float* var, float* O, float* A,
                       float* LP, float* V, float* R, float* D, float* Vlast, const float* act_noise,
                       const float* reset_noise) {
  EnvState* E = (EnvState*)h;
  int dev = 0;
  HIPCHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices || !scratch_addr[dev]) {
    fprintf(stderr, "g1_rollout_noalloc: no env was created on the current device\n");
    return -1;
  }
  long total = 0;
  make_packed(E->shape, nullptr, nullptr, &total);
  if (total > kScratchFloats) {
    fprintf(stderr, "g1_rollout_noalloc: the packed policy needs %ld floats, the scratch holds %ld\n", total,
            kScratchFloats);
    return -1;
  }
  rollout_impl(E, H, W, mean, var, O, A, LP, V, R, D, Vlast, act_noise, reset_noise, scratch_addr[dev], kScratchFloats);
  return 0;
}

void g1_env_bench_phys(void* h, int K) {
  EnvState* E = (EnvState*)h;
  poll_queue_error(E);
  if (K <= 0) return;   // no control step (the reference's loop runs zero times)
  PhysArgs pa = phys_args(E);
  pa.K = K; pa.act = E->zero_act; pa.t0 = 0; pa.astep = 0; pa.rstep = 0; pa.R = E->bench_r; pa.D = E->bench_d;
  launch_physics(E, pa);
  HIPCHECK(hipDeviceSynchronize());
  check_queue(E);
}

void g1_env_qpos(void* h, float* out) {
  EnvState* E = (EnvState*)h;
  HIPCHECK(hipMemcpy(out, E->qp, (size_t)kNQ * 4, hipMemcpyDeviceToHost));
  check_queue(E);
}

void g1_env_qpos_all(void* h, float* out) {
  EnvState* E = (EnvState*)h;
  HIPCHECK(hipMemcpy(out, E->qp, (size_t)E->N * kNQ * 4, hipMemcpyDeviceToHost));
  check_queue(E);
}

void g1_occupancy_report(void) {
  int dev = 0;
  HIPCHECK(hipGetDevice(&dev));
  hipDeviceProp_t p;
  HIPCHECK(hipGetDeviceProperties(&p, dev));
  printf("%s (%s): %d CUs, LDS/block %zu B, regs/block %d\n", p.name, p.gcnArchName, p.multiProcessorCount,
         p.sharedMemPerBlock, p.regsPerBlock);
  struct { const char* nm; const void* fn; int threads; size_t smem; } ks[] = {
      {"k_rollout", rollout_kernel_fn(false), kPhysThreads, 0},
      {"k_rollout (wide)", rollout_kernel_fn(true), kPhysThreads, 0},
      {"k_physics", (const void*)k_physics, kPhysThreads, 0},
      {"k_policy", (const void*)k_policy, kPolicyThreads, policy_smem(PolicyShape{2, {256, 256, 0, 0}, 0})},
      {"k_probe", (const void*)k_probe, kPhysThreads, 0}};
  for (auto& k : ks) {
    hipFuncAttributes fa;
    HIPCHECK(hipFuncGetAttributes(&fa, k.fn));
    int mb = 0;
    HIPCHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&mb, k.fn, k.threads, k.smem));
    printf("  %-17s regs=%d scratch=%zuB lds=%zuB maxBlocks/CU=%d waves/CU=%d\n", k.nm, fa.numRegs, fa.localSizeBytes,
           fa.sharedSizeBytes + k.smem, mb, mb * k.threads / 64);
  }
}

// ---- additive exports (no counterpart in the reference ABI) --------------------------------
void g1_env_set_state(void* h, const float* qp, const float* qv, const float* pa, const int* steps) {
  EnvState* E = (EnvState*)h;
  poll_queue_error(E);
  const size_t N = E->N;
  HIPCHECK(hipMemcpy(E->qp, qp, N * kNQ * 4, hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(E->qv, qv, N * kNV * 4, hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(E->pa, pa, N * kAct * 4, hipMemcpyHostToDevice));
  HIPCHECK(hipMemcpy(E->steps, steps, N * 4, hipMemcpyHostToDevice));
}

void g1_env_get_state(void* h, float* qp, float* qv, float* pa, int* steps) {
  EnvState* E = (EnvState*)h;
  const size_t N = E->N;
  HIPCHECK(hipMemcpy(qp, E->qp, N * kNQ * 4, hipMemcpyDeviceToHost));
  HIPCHECK(hipMemcpy(qv, E->qv, N * kNV * 4, hipMemcpyDeviceToHost));
  HIPCHECK(hipMemcpy(pa, E->pa, N * kAct * 4, hipMemcpyDeviceToHost));
  HIPCHECK(hipMemcpy(steps, E->steps, N * 4, hipMemcpyDeviceToHost));
  check_queue(E);
}

int g1_env_set_policy(void* h, int nlayers, const int* hidden, int activation) {
  EnvState* E = (EnvState*)h;
  if (nlayers < 1 || nlayers > kMaxLayers - 1 || (activation != 0 && activation != 1)) {
    fprintf(stderr, "g1_env_set_policy: need 1..%d hidden layers and activation 0 (tanh) or 1 (ELU)\n", kMaxLayers - 1);
    return -1;
  }
  PolicyShape sh{nlayers, {0, 0, 0, 0}, activation};
  for (int i = 0; i < nlayers; ++i) {
    if (hidden[i] < 1 || hidden[i] > kMaxHidden) {
      fprintf(stderr, "g1_env_set_policy: hidden width must be in 1..%d\n", kMaxHidden);
      return -1;
    }
    sh.hid[i] = hidden[i];
  }
  E->shape = sh;
  return 0;
}

long g1_env_device_bytes(void* h) { return ((EnvState*)h)->dev_bytes; }

long g1_env_policy_params(void* h) { return policy_param_count(((EnvState*)h)->shape); }

void g1_env_set_contact(void* h, float mu, int pgs_iters) {
  EnvState* E = (EnvState*)h;
  if (!(mu >= 0.f) || pgs_iters < 0) fail("g1_env_set_contact: invalid mu/pgs_iters");
  E->mu = mu;
  E->pgs = pgs_iters;
}

void g1_env_ncon_hist(void* h, int enable, unsigned long long* out9) {
  EnvState* E = (EnvState*)h;
  if (out9) HIPCHECK(hipMemcpy(out9, E->ncon_hist, 9 * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  check_queue(E);
  HIPCHECK(hipMemset(E->ncon_hist, 0, 9 * sizeof(unsigned long long)));
  E->hist_on = enable;
}

void g1_env_profile(void* h, int enable) {
  EnvState* E = (EnvState*)h;
  E->prof_on = enable;
  E->n_phys = E->n_pol = 0;
}

void g1_env_profile_read(void* h, double* out4) {
  EnvState* E = (EnvState*)h;
  HIPCHECK(hipDeviceSynchronize());
  check_queue(E);
  double tp = 0.0, tq = 0.0;
  for (size_t i = 0; i + 1 < E->n_phys; i += 2) {
    float ms = 0.f;
    HIPCHECK(hipEventElapsedTime(&ms, E->ev_phys[i], E->ev_phys[i + 1]));
    tp += ms;
  }
  for (size_t i = 0; i + 1 < E->n_pol; i += 2) {
    float ms = 0.f;
    HIPCHECK(hipEventElapsedTime(&ms, E->ev_pol[i], E->ev_pol[i + 1]));
    tq += ms;
  }
  out4[0] = tp; out4[1] = (double)(E->n_phys / 2); out4[2] = tq; out4[3] = (double)(E->n_pol / 2);
}

int g1_env_check(void* h) {
  EnvState* E = (EnvState*)h;
  HIPCHECK(hipDeviceSynchronize());
  int err = 0;
  HIPCHECK(hipMemcpy(&err, E->qerr, sizeof(int), hipMemcpyDeviceToHost));
  return err;
}

int g1_env_set_fused(void* h, int on) {
  EnvState* E = (EnvState*)h;
  if (on != 0 && on != 1) return -1;
  E->fused = on;
  return (on && !fused_shape(E->shape, false)) ? 1 : 0;
}

int g1_env_set_handover(void* h, int fences) {
  EnvState* E = (EnvState*)h;
  if (fences != 0 && fences != 1) return -1;
  if (!fences && !E->xlocal) return -1;   // the L2 hand-over needs the round-robin placement
  E->fences = fences;
  return 0;
}

void g1_probe_qacc(int n, float* qpos, float* qvel, const float* tau, int damped, int contact, int pgs, float mu,
                   float* qacc, int* ncon) {
  if (n <= 0) return;
  ProbeArgs a{};
  a.n = n; a.mode = 0; a.qp = qpos; a.qv = qvel; a.tau = tau; a.qacc = qacc; a.ncon = ncon;
  a.pgs = pgs; a.damped = damped; a.contact = contact; a.guard = 0; a.nsub = 1; a.mu = mu;
  hipLaunchKernelGGL(k_probe, dim3((n + 1) / 2), dim3(kPhysThreads), 0, 0, a);
  HIPCHECK(hipGetLastError());
}

void g1_probe_substep(int n, float* qpos, float* qvel, const float* target, int nsub, int pgs, float mu, float* qacc,
                      int* ncon) {
  if (n <= 0) return;
  ProbeArgs a{};
  a.n = n; a.mode = 1; a.qp = qpos; a.qv = qvel; a.target = target; a.qacc = qacc; a.ncon = ncon;
  a.pgs = pgs; a.damped = 1; a.contact = 1; a.guard = 1; a.nsub = nsub; a.mu = mu;
  hipLaunchKernelGGL(k_probe, dim3((n + 1) / 2), dim3(kPhysThreads), 0, 0, a);
  HIPCHECK(hipGetLastError());
}

void g1_dynamics_bench(int n, float* qpos, float* qvel, const float* tau, int nsub, int contact, int damped, int guard,
                       int pgs, float mu, float* qacc, int* ncon) {
  if (n <= 0 || nsub <= 0) return;
  ProbeArgs a{};
  a.n = n; a.mode = 2; a.qp = qpos; a.qv = qvel; a.tau = tau; a.qacc = qacc; a.ncon = ncon;
  a.pgs = pgs; a.damped = damped; a.contact = contact; a.guard = guard; a.nsub = nsub; a.mu = mu;
  hipLaunchKernelGGL(k_probe, dim3((n + 1) / 2), dim3(kPhysThreads), 0, 0, a);
  HIPCHECK(hipGetLastError());
}

int g1_probe_policy(int n, int nlayers, const int* hidden, int activation, const float* W, const float* obs_norm,
                    float* mu_out, float* v_out) {
  if (n <= 0) return 0;
  EnvState tmp{};
  tmp.N = n;
  if (g1_env_set_policy(&tmp, nlayers, hidden, activation) != 0) return -1;
  PackedPolicy pp;
  pack_policy(&tmp, W, &pp);
  PolicyArgs a{};
  a.N = n; a.t = 0; a.H = 1; a.pp = pp; a.shape = tmp.shape; a.obs_in = obs_norm; a.mu_out = mu_out; a.V = v_out;
  a.ldx = policy_ldx(tmp.shape);
  launch_policy_kernel(a, n, tmp.shape);
  HIPCHECK(hipDeviceSynchronize());
  HIPCHECK(hipFree(tmp.Wp));
  return 0;
}

void g1_probe_divide(int n, const float* a, const float* b, float* rcp, float* quot) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_divide, dim3((n + 255) / 256), dim3(256), 0, 0, a, b, rcp, quot, n);
  HIPCHECK(hipGetLastError());
}

void g1_probe_sqrt(int n, const float* x, float* out) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_sqrt, dim3((n + 255) / 256), dim3(256), 0, 0, x, out, n);
  HIPCHECK(hipGetLastError());
}

void g1_probe_sincos(int n, const float* x, float* sn, float* cs) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_sincos, dim3((n + 255) / 256), dim3(256), 0, 0, x, sn, cs, n);
  HIPCHECK(hipGetLastError());
}

void g1_probe_sincos_hinge(int n, const float* x, float* sn, float* cs) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_sincos_hinge, dim3((n + 255) / 256), dim3(256), 0, 0, x, sn, cs, n);
  HIPCHECK(hipGetLastError());
}

void g1_probe_philox(int n, const unsigned* ctr, unsigned* out, unsigned k0, unsigned k1) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_philox, dim3((n + 255) / 256), dim3(256), 0, 0, ctr, out, n, k0, k1);
  HIPCHECK(hipGetLastError());
}

}  // extern "C"
