// rollout.h -- the policy of one 16-world tile on one wave, for the single-launch rollout (k_rollout).
//
// The persistent physics kernel also runs the policy: when the 8 world pairs of a tile have
// finished control step t, one wave computes observation, normalisation, MLP, sampling and
// log-probability for the tile's 16 worlds, and the pairs' next physics items start from its
// actions. The MLP runs on v_mfma_f32_16x16x4f32 with the weights as the A operand and the
// activations as the B operand: lane l holds world j = l % 16 throughout, as input feature group
// g = l / 16 for a B operand and as output rows 4g..4g+3 of a 16-row tile in the accumulator
// (D[4 (l / 16) + v][l % 16] in register v). A layer's accumulator registers are therefore the
// next layer's B operands without any data movement, provided the next layer's K dimension is
// taken in that order: k-step s of a layer after the first reads input neuron
// kappa(s, g) = 16 (s / 4) + 4 g + s % 4 (the first layer reads observation feature 4 s + g). The
// weights are packed to match (k_pack_tiles), so each lane's operands of four k-steps are one
// float4 load and the 64 lanes of one load read one contiguous 1 KB line.
//
// Reference: obs src/g1_env.cu:46-81; normalise/clamp :298-302; MLP :219-239 (the AC of
// scripts/ppo.py:85-99, packing scripts/ppo_fused.py:35-44); sampling + log-prob :308-318.
#pragma once
#include <hip/hip_runtime.h>

#include "policy.h"

namespace g1k {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTilePairs = 8;                  // world pairs per policy tile (one queue's pairs)
constexpr int kTileW = 2 * kTilePairs;         // 16 worlds: the N dimension of the 16x16x4 MFMA
constexpr int kTileMaxHidden = 256;            // widest hidden layer of the one-launch rollout
constexpr int kTileMaxT = kTileMaxHidden / 16; // 16-row output tiles of the widest layer
constexpr int kObsSteps = 28;                  // k-steps of the first layer: 100 features, padded to 112
constexpr int kHeadT = 2;                      // head rows: mu 0..28, value 29, 30..31 zero

// Packed layout of a two-hidden-layer policy for the tile MLP (floats, offsets into one buffer):
// layer L's weights as [T][s / 4][lane][s % 4] (T: 16-row output tile, s: k-step), then its bias in
// natural row order padded to whole tiles; the log standard deviation (29 values + 3 zeros); last
// the observation normalisation as [3][g][s] for feature 4 s + g: mean, d = RN(sqrt(var + 1e-8))
// and RN(1 / d) (features past 100: 0, 1, 1), so that lane group g reads its own as float4s.
struct TileLayout {
  int nT[3];        // output tiles of layer 0, layer 1, head
  int nQ[3];        // k-step quads of layer 0, layer 1, head
  long woff[3], boff[3];
  long ls_off;
  long nrm_off;
  long total;
  int act;          // 0 tanh, 1 ELU
};

// Every layer is laid out at the widest shape (256-256): rows past a layer's width and k-steps past
// its input width hold zeros.
__host__ __device__ inline TileLayout tile_layout(int act) {
  TileLayout t{};
  t.nT[0] = kTileMaxT; t.nT[1] = kTileMaxT; t.nT[2] = kHeadT;
  t.nQ[0] = kObsSteps / 4; t.nQ[1] = kTileMaxT; t.nQ[2] = kTileMaxT;
  long off = 0;
  for (int L = 0; L < 3; ++L) {
    t.woff[L] = off;
    off += (long)t.nT[L] * t.nQ[L] * 64 * 4;
    t.boff[L] = off;
    off += (long)t.nT[L] * 16;
  }
  t.ls_off = off;
  t.nrm_off = off + 32;
  t.total = t.nrm_off + 3 * 4 * kObsSteps;
  t.act = act;
  return t;
}

// Input feature read by k-step s, lane group g of layer L.
__host__ __device__ __forceinline__ int tile_kappa(int L, int s, int g) {
  return L == 0 ? 4 * s + g : 16 * (s >> 2) + 4 * g + (s & 3);
}

// Packed layout of a policy of 1..3 hidden layers of at most 512 units (any activation) for the
// wide tile (policy_tile_wide), in floats: per layer L (the head last) the weights as
// [T][q][lane][4] (T: 16-row output tile, q: k-quad of four k-steps, lane (row j = lane mod 16,
// group g = lane / 16) holds W[16 T + j][kappa(L, 4 q + e, g)] in element e) and the bias in
// natural row order; then the log standard deviation and the normalisation constants as in
// TileLayout. A hidden layer's output tiles are padded to a multiple of kWideGroup (zero rows:
// act(0) = 0 adds exact zeros downstream); the head has kHeadT tiles (mu 0..28, value 29).
constexpr int kWideMaxLayers = 4;   // hidden layers + head
constexpr int kWideGroup = 4;       // output tiles a wave accumulates at once (independent chains)
struct WideLayout {
  int nl;                           // hidden layers (1..3)
  int nT[kWideMaxLayers];           // output tiles of layer L
  int nQ[kWideMaxLayers];           // k-quads of layer L (layer 0: the observation's kObsSteps / 4)
  long woff[kWideMaxLayers], boff[kWideMaxLayers];
  long ls_off, nrm_off, total;
  int maxT;                         // output tiles of the widest hidden layer
  int act;                          // 0 tanh, 1 ELU
};

static_assert(kWideGroup % 4 == 0, "hidden layers feed the next layer a multiple of 4 k-quads");
__host__ __device__ inline WideLayout wide_layout(int nl, const int* hid, int act) {
  WideLayout t{};
  t.nl = nl;
  t.act = act;
  long off = 0;
  for (int L = 0; L <= nl; ++L) {
    t.nT[L] = L < nl ? (hid[L] + 16 * kWideGroup - 1) / (16 * kWideGroup) * kWideGroup : kHeadT;
    t.nQ[L] = L == 0 ? kObsSteps / 4 : t.nT[L - 1];
    t.woff[L] = off;
    off += (long)t.nT[L] * t.nQ[L] * 64 * 4;
    t.boff[L] = off;
    off += (long)t.nT[L] * 16;
    if (L < nl && t.nT[L] > t.maxT) t.maxT = t.nT[L];
  }
  t.ls_off = off;
  t.nrm_off = off + 32;
  t.total = t.nrm_off + 3 * 4 * kObsSteps;
  return t;
}

struct TileArgs {
  const float* Wt;          // packed (TileLayout, or WideLayout when wide)
  TileLayout tl;
  const float* act_noise;   // [H][N][29] or null (Philox)
  float* O; float* A; float* LP; float* V; float* Vlast;
  int H;
  int wide;                 // 1: the wide tile (policy_tile_wide) on WideLayout wl
  WideLayout wl;
  float* scr;               // wide tile: per block, two activation buffers of wl.maxT * 256 floats
};

// The 16 worlds of tile u of queue q: pairs p = q + 32 (8 u + i), i < 8, worlds 2p and 2p + 1;
// world slot j holds pair i = j / 2, world 2p + (j & 1).
__device__ __forceinline__ int tile_world(int q, int u, int j, int queues) {
  const int p = q + queues * (kTilePairs * u + (j >> 1));
  return 2 * p + (j & 1);
}

__device__ __forceinline__ f32x4 mfma4(f32x4 w, const float* x, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w.x, x[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w.y, x[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w.z, x[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w.w, x[3], acc, 0, 0, 0);
  return acc;
}

constexpr int kObsLoads = 25;   // k-steps of the first layer that read a state value (4 s + g < 100)

// Observation feature i (reference: src/g1_env.cu:69-81): base angular and linear velocity (qvel
// 0..5), gravity in the base frame (from the base quaternion), joint positions (qpos 7..35), joint
// velocities (qvel 6..34), previous action, the command (0.8) and three zeros. obs_src gives the
// state value feature i copies (a valid address for the others, whose value obs_value forms).
__device__ __forceinline__ const float* obs_src(const float* qp, const float* qv, const float* pa, int i) {
  const float* p = qv;
  p = i < 6 ? qv + i : p;
  p = (i >= 9 && i < 38) ? qp + (i - 2) : p;
  p = (i >= 38 && i < 67) ? qv + (i - 32) : p;
  p = (i >= 67 && i < 96) ? pa + (i - 67) : p;
  return p;
}
__device__ __forceinline__ float obs_value(float raw, float qw, float qx, float qy, float qz, int i) {
  if (i >= 6 && i < 9) {
    const float r = (i == 6)   ? 2.f * __builtin_fmaf(-qw, qy, qx * qz)
                    : (i == 7) ? 2.f * __builtin_fmaf(qw, qx, qy * qz)
                               : __builtin_fmaf(-2.f, __builtin_fmaf(qy, qy, qx * qx), 1.f);
    return -r;
  }
  if (i >= 96) return i == 96 ? 0.8f : 0.f;
  return raw;
}

constexpr int kTileLds = kTileW * 32 + 2 * kTileMaxHidden;   // LDS floats of one tile's policy

// ---- observation (raw to O, reference: src/g1_env.cu:69-81) and frozen normalisation (:298-302)
// of a tile's worlds: lane (j, g) forms features 4 s + g of its world, the first layer's B
// operands x[s]. Every state value is loaded first (one load per feature, all in flight together),
// then the normalisation constants (nrm: [3][4][kObsSteps] as packed by the tile layouts).
template <class LoadT>
__device__ __forceinline__ void tile_observation(const TileArgs& a, const float* nrm, const float* qpos,
                                                 const float* qvel, const float* pact, int N, int t, int w,
                                                 bool valid, int lane, LoadT ld, float (&x)[kObsSteps]) {
  const int g = (lane >> 4) & 3;   // (& 3: the lane arrives through an opaque asm; with g's range known
                                   // the feature tests of obs_value fold for every quad but three)
  const int wc = valid ? w : N - 1;
  const float* qp = qpos + (long)wc * kNQ;
  const float* qv = qvel + (long)wc * kNV;
  const float* pa = pact + (long)wc * kAct;
  const float qw = ld(qp + 3), qx = ld(qp + 4), qy = ld(qp + 5), qz = ld(qp + 6);
  // Feature k = 4 s + g comes from one array for every lane of a quad s except at the array
  // boundaries (s = 1, 2, 9, 16): one lane-dependent base per array (qv[k], qp[k - 2], qv[k - 32],
  // pa[k - 67]) with the quad's offset as an immediate keeps the addresses at one register per
  // array; the boundary quads load both candidates at in-range indices and select per lane.
  // (Lanes whose feature is computed, not loaded, take an unused in-range value.)
  float raw[kObsLoads];
  const float* const fv = qv + g;
  const float* const fq = qp + g - 2;
  const float* const fw = qv + g - 32;
  const float* const fa = pa + g - 67;
#pragma unroll
  for (int s = 0; s < kObsLoads; ++s) {
    const int k0 = 4 * s;
    if (k0 + 3 < 6) raw[s] = ld(fv + k0);                                  // qvel 0..5
    else if (k0 < 9) raw[s] = k0 + g < 9 ? ld(qv + (g < 2 ? 4 + g : 0)) : ld(fq + k0);   // qvel 4, 5 | gravity | qpos
    else if (k0 + 3 < 38) raw[s] = ld(fq + k0);                            // qpos 7..35
    else if (k0 < 38) {                                                    // qpos 34, 35 | qvel 6, 7
      const float a = ld(qp + (g < 2 ? k0 + g - 2 : 0)), b = ld(qv + (g < 2 ? 0 : k0 + g - 32));
      raw[s] = g < 2 ? a : b;
    } else if (k0 + 3 < 67) raw[s] = ld(fw + k0);                          // qvel 6..34
    else if (k0 < 67) {                                                    // qvel 32..34 | prev action 0
      const float a = ld(qv + (k0 + g < 67 ? k0 + g - 32 : 0)), b = ld(pa + (k0 + g < 67 ? 0 : k0 + g - 67));
      raw[s] = k0 + g < 67 ? a : b;
    } else if (k0 + 3 < 96) raw[s] = ld(fa + k0);                          // prev action 1..28
    else raw[s] = ld(fv);                                                  // command and padding (unused)
  }
  const float4* NC = reinterpret_cast<const float4*>(nrm + kObsSteps * g);
  float4 nmean[kObsSteps / 4], ndiv[kObsSteps / 4], nrcp[kObsSteps / 4];
#pragma unroll
  for (int q = 0; q < kObsSteps / 4; ++q) {
    nmean[q] = NC[q];
    ndiv[q] = NC[q + kObsSteps];
    nrcp[q] = NC[q + 2 * kObsSteps];
  }
#pragma unroll
  for (int s = 0; s < kObsSteps; ++s) {
    const int k = 4 * s + g;
    float z = 0.f;
    if (s < kObsLoads) {
      const float o = obs_value(raw[s], qw, qx, qy, qz, k);
      if (valid && t < a.H) a.O[((long)t * N + w) * kObs + k] = o;
      const float m = (&nmean[s >> 2].x)[s & 3], d = (&ndiv[s >> 2].x)[s & 3], y = (&nrcp[s >> 2].x)[s & 3];
      z = div_rn_inf(o - m, d, y);
      if (z < -10.f) z = -10.f; else if (z > 10.f) z = 10.f;
    }
    x[s] = z;
  }
}

// ---- the tile's outputs from the head's accumulators hd (rows 4 g + v of head tile ht in lane
// (j, g), register v): the value (head row 29), then for t < H the sampling and log-prob
// (reference: src/g1_env.cu:308-318): lane g owns actions 4g..4g+3 and 16+4g..16+4g+3, i.e. the
// action pairs 2g, 2g+1, 8+2g, 9+2g; both Box-Muller normals of one Philox counter go to the actions
// of one pair. The log-prob terms go through LDS (lds: kTileW x 32 floats) so that one lane sums
// each world's 29 terms in action order.
template <class LoadT>
__device__ __forceinline__ void tile_outputs(const TileArgs& a, const f32x4 (&hd)[kHeadT], const float* ls,
                                             const unsigned* rngc, unsigned long long seed, int N, int t, int w,
                                             bool valid, int lane, float* lds, LoadT ld) {
  const int j = lane & 15, g = (lane >> 4) & 3;
  const int wc = valid ? w : N - 1;
  // ---- value (head row 29: tile 1, rows 4 g + v with g = 3, v = 1)
  if (g == 3 && valid) {
    if (t == a.H) a.Vlast[w] = hd[1][1];
    else a.V[(long)t * N + w] = hd[1][1];
  }
  if (t == a.H) return;
  const float LOG2PI = 1.8378770664093453f;
  const unsigned rng = valid ? ld(rngc + wc) : 0u;
  const long ab = ((long)t * N + w) * kAct;
#pragma unroll
  for (int ht = 0; ht < kHeadT; ++ht) {
#pragma unroll
    for (int hp = 0; hp < 2; ++hp) {
      const int i0 = 16 * ht + 4 * g + 2 * hp;   // actions i0, i0 + 1
      if (i0 < kAct) {
        float nz[2];
        if (a.act_noise) {
          nz[0] = valid ? a.act_noise[ab + i0] : 0.f;
          nz[1] = (valid && i0 + 1 < kAct) ? a.act_noise[ab + i0 + 1] : 0.f;
        } else {
          rng_normal2(seed, wc, rng, kStreamAction, i0 >> 1, nz[0], nz[1]);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int i = i0 + e;
          if (i < kAct) {
            const float lsi = ls[i];
            if (valid) a.A[ab + i] = hd[ht][2 * hp + e] + expf(lsi) * nz[e];
            lds[j * 32 + i] = -0.5f * nz[e] * nz[e] - lsi - 0.5f * LOG2PI;
          }
        }
      }
    }
  }
  __syncthreads();
  if (g == 0 && valid) {
    float lpsum = 0.f;
    for (int i = 0; i < kAct; ++i) lpsum += lds[j * 32 + i];
    a.LP[(long)t * N + w] = lpsum;
  }
  __syncthreads();
}

// Policy of control step t (t == H: the bootstrap value only) for the tile's worlds w_j, given by
// the caller (valid: w_j < N), on the fixed 256-256 shape of TileLayout. State is read with `ld`
// (from the L2: other waves of the launch wrote it). hid: LDS scratch of kTileLds floats: the
// log-prob terms (kTileW x 32), then the two layers' biases.
template <int ACT, class LoadT>
__device__ __forceinline__ void policy_tile(const TileArgs& a, const float* qpos, const float* qvel, const float* pact,
                                            const unsigned* rngc, unsigned long long seed, int N, int t, int w,
                                            bool valid, float* hid, LoadT ld) {
  // the lane index goes through an opaque asm so that nothing derived from it is hoisted out of the
  // caller's item loop (where it would stay live beside the physics items' registers)
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));
  const int g = (lane >> 4) & 3;
  const TileLayout& T = a.tl;
  float x[kObsSteps];
  tile_observation(a, a.Wt + T.nrm_off, qpos, qvel, pact, N, t, w, valid, lane, ld, x);

  // ---- the MLP, on the fixed 256-256 shape (narrower layers are padded with zero weights and
  // biases, whose rows give act(0) = 0 and add exact zeros downstream). Layer 0 runs in 16 output
  // tiles, fully unrolled: tile T's activations (rows 16 T + 4 g + v of world j in lane (j, g),
  // register v) are the second layer's B operands of k-quad T as they stand, so the hidden
  // activations never leave the registers. Weights stream from the L2 through register slots ahead
  // of their MFMAs, every load on every path (waits then count only older loads); the biases are
  // read from LDS.
  float* hb0 = hid + kTileW * 32;
  float* hb1 = hb0 + kTileMaxHidden;
  *reinterpret_cast<float4*>(hb0 + 4 * lane) = *reinterpret_cast<const float4*>(a.Wt + T.boff[0] + 4 * lane);
  *reinterpret_cast<float4*>(hb1 + 4 * lane) = *reinterpret_cast<const float4*>(a.Wt + T.boff[1] + 4 * lane);
  constexpr int kQ0 = kObsSteps / 4;            // k-quads per output tile of layer 0
  constexpr int kQ0All = kTileMaxT * kQ0;        // layer 0's k-quads in storage order
  constexpr int kRing0 = 8, kAhead0 = kQ0;       // quad slots; a quad is loaded one tile ahead
  const float4* W0 = reinterpret_cast<const float4*>(a.Wt + T.woff[0]);
  float4 w0[kRing0];
#pragma unroll
  for (int gq = 0; gq < kAhead0; ++gq) {
    w0[gq % kRing0] = W0[gq * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();   // the biases are in LDS
  f32x4 h[kTileMaxT];
#pragma unroll
  for (int ot = 0; ot < kTileMaxT; ++ot) {
    const float4 bv = *reinterpret_cast<const float4*>(hb0 + 16 * ot + 4 * g);
    f32x4 acc = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
    for (int qd = 0; qd < kQ0; ++qd) {
      const int gq = ot * kQ0 + qd;
      if (gq + kAhead0 < kQ0All) w0[(gq + kAhead0) % kRing0] = W0[(gq + kAhead0) * 64 + lane];
      const float4 wq = w0[gq % kRing0];
      acc = mfma4(f32x4{wq.x, wq.y, wq.z, wq.w}, x + 4 * qd, acc);
      __builtin_amdgcn_sched_barrier(0);   // each refill issued ahead of its quad's MFMAs, as written
    }
    h[ot] = f32x4{act_tile<ACT>(acc[0]), act_tile<ACT>(acc[1]), act_tile<ACT>(acc[2]), act_tile<ACT>(acc[3])};
    __builtin_amdgcn_sched_barrier(0);   // keep each tile's loads and MFMAs within the tile
  }

  // ---- layer 1 tile by tile, each tile's activations fed into the head as its k-quad; the weights
  // in 4-quad blocks through two slots, each refilled with the block after next as soon as its
  // block's MFMAs are issued
  const float4* W1 = reinterpret_cast<const float4*>(a.Wt + T.woff[1]);
  const float4* Wh = reinterpret_cast<const float4*>(a.Wt + T.woff[2]);
  f32x4 hd[kHeadT];
#pragma unroll
  for (int ht = 0; ht < kHeadT; ++ht) {
    const float4 bv = *reinterpret_cast<const float4*>(a.Wt + T.boff[2] + 16 * ht + 4 * g);
    hd[ht] = f32x4{bv.x, bv.y, bv.z, bv.w};
  }
  float4 wr[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wr[qb][i] = W1[(4 * qb + i) * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll 1
  for (int ot = 0; ot < kTileMaxT; ++ot) {
    const int on = ot + 1 < kTileMaxT ? ot + 1 : ot;   // the last tile reloads itself
    float4 wh[kHeadT];
#pragma unroll
    for (int ht = 0; ht < kHeadT; ++ht) wh[ht] = Wh[(ht * kTileMaxT + ot) * 64 + lane];
    const float4 bv = *reinterpret_cast<const float4*>(hb1 + 16 * ot + 4 * g);
    f32x4 acc = {bv.x, bv.y, bv.z, bv.w};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 hq = h[4 * qb + i];
        const float xb[4] = {hq[0], hq[1], hq[2], hq[3]};
        acc = mfma4(f32x4{wr[qb & 1][i].x, wr[qb & 1][i].y, wr[qb & 1][i].z, wr[qb & 1][i].w}, xb, acc);
      }
      // block qb + 2 of this tile, or block qb - 2 of the next
      const int nb = qb < 2 ? 4 * ot + qb + 2 : 4 * on + qb - 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) wr[qb & 1][i] = W1[(4 * nb + i) * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);   // the refill issued here, a block ahead of its use
    }
    const float h2[4] = {act_tile<ACT>(acc[0]), act_tile<ACT>(acc[1]), act_tile<ACT>(acc[2]), act_tile<ACT>(acc[3])};
#pragma unroll
    for (int ht = 0; ht < kHeadT; ++ht) hd[ht] = mfma4(f32x4{wh[ht].x, wh[ht].y, wh[ht].z, wh[ht].w}, h2, hd[ht]);
  }
  tile_outputs(a, hd, a.Wt + T.ls_off, rngc, seed, N, t, w, valid, lane, hid, ld);
}

// One layer of the wide tile: nT output tiles over nQ k-quads of B operands (in: this lane's float4
// per quad, the previous layer's outputs; layer 0 (kFromRegs): the observation x in registers), G
// output tiles at a time, each tile's four k-steps interleaved with the other tiles' (G independent
// accumulation chains). Layer 0 loads quad q + 2 after quad q's MFMAs (two register sets); the
// other layers load quad q + 4 (four register sets, the quad loop unrolled by four), so a quad's
// loads have three quads of MFMAs (3 x G x 4 x 32 cycles) to arrive. Outputs (activated) go to
// out[T * 64 + lane], or (kHead, nT = G = kHeadT) into hd. (the scheduling pins keep each quad's
// loads together and in program order, so that a wait for one register set counts only the loads
// issued before the later sets'; without them the compiler hoists every load of the unrolled body
// to its top, past the 256-VGPR budget)
template <int G>
__device__ __forceinline__ void wide_load(const float4* Wg, int nQ, int q, const float4* in, int lane, float4 (&w)[G],
                                          float4& x, bool kFromRegs) {
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < G; ++i) w[i] = Wg[((long)i * nQ + q) * 64];
  if (!kFromRegs) x = in[q * 64 + lane];
  __builtin_amdgcn_sched_barrier(0);
}
template <int G>
__device__ __forceinline__ void wide_mfma(const float4 (&w)[G], const float (&xb)[4], f32x4 (&acc)[G]) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int i = 0; i < G; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32((&w[i].x)[e], xb[e], acc[i], 0, 0, 0);
}
template <int ACT, int G, bool kFromRegs, bool kHead>
__device__ __forceinline__ void wide_layer(const float4* W, const float* bias, int nT, int nQ, const float4* in,
                                           const float (&x)[kObsSteps], float4* out, f32x4 (&hd)[kHeadT], int lane) {
  const int g = (lane >> 4) & 3;
#pragma unroll 1
  for (int T0 = 0; T0 < nT; T0 += G) {
    f32x4 acc[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const float4 bv = *reinterpret_cast<const float4*>(bias + 16 * (T0 + i) + 4 * g);
      acc[i] = f32x4{bv.x, bv.y, bv.z, bv.w};
    }
    const float4* Wg = W + (long)T0 * nQ * 64 + lane;
    float4 wa[G], wb[G], xa = {0.f, 0.f, 0.f, 0.f}, xb = {0.f, 0.f, 0.f, 0.f};
    wide_load<G>(Wg, nQ, 0, in, lane, wa, xa, kFromRegs);
    wide_load<G>(Wg, nQ, 1, in, lane, wb, xb, kFromRegs);
    if (kFromRegs) {
      // layer 0: the observation quads in registers, the quad loop fully unrolled
      constexpr int nq0 = kObsSteps / 4;
#pragma unroll
      for (int q = 0; q < nq0; ++q) {
        float4 (&wc)[G] = (q & 1) ? wb : wa;
        const float xs[4] = {x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]};
        wide_mfma<G>(wc, xs, acc);
        if (q + 2 < nq0) wide_load<G>(Wg, nQ, q + 2, in, lane, wc, xa, true);
      }
    } else {
      // four register sets, each reloaded with the quad four ahead once its MFMAs are issued; nQ is
      // a multiple of 4 (a hidden layer's output tiles are padded to a multiple of kWideGroup), so
      // the loop body is four whole quads with no exit between them
      float4 wc[G], wd[G], xc = {0.f, 0.f, 0.f, 0.f}, xd = {0.f, 0.f, 0.f, 0.f};
      wide_load<G>(Wg, nQ, 2, in, lane, wc, xc, false);
      wide_load<G>(Wg, nQ, 3, in, lane, wd, xd, false);
#pragma unroll 1
      for (int q = 0; q < nQ; q += 4) {
        const float xs0[4] = {xa.x, xa.y, xa.z, xa.w};
        wide_mfma<G>(wa, xs0, acc);
        wide_load<G>(Wg, nQ, q + 4 < nQ ? q + 4 : nQ - 1, in, lane, wa, xa, false);   // the tail reloads
        const float xs1[4] = {xb.x, xb.y, xb.z, xb.w};
        wide_mfma<G>(wb, xs1, acc);
        wide_load<G>(Wg, nQ, q + 5 < nQ ? q + 5 : nQ - 1, in, lane, wb, xb, false);
        const float xs2[4] = {xc.x, xc.y, xc.z, xc.w};
        wide_mfma<G>(wc, xs2, acc);
        wide_load<G>(Wg, nQ, q + 6 < nQ ? q + 6 : nQ - 1, in, lane, wc, xc, false);
        const float xs3[4] = {xd.x, xd.y, xd.z, xd.w};
        wide_mfma<G>(wd, xs3, acc);
        wide_load<G>(Wg, nQ, q + 7 < nQ ? q + 7 : nQ - 1, in, lane, wd, xd, false);
      }
    }
    if (kHead) {
#pragma unroll
      for (int i = 0; i < G; ++i) hd[i] = acc[i];
    } else {
#pragma unroll
      for (int i = 0; i < G; ++i)
        out[(T0 + i) * 64 + lane] = float4{act_tile<ACT>(acc[i][0]), act_tile<ACT>(acc[i][1]),
                                           act_tile<ACT>(acc[i][2]), act_tile<ACT>(acc[i][3])};
    }
  }
}

// Policy of control step t for the tile's worlds on a policy of 1..3 hidden layers of at most 512
// units (WideLayout), for k_rollout: layer by layer on v_mfma_f32_16x16x4f32 with the weights as A
// operands and the activations as B operands (lane (j, g): world j, input group g), kWideGroup
// output tiles at a time. A layer's activated outputs go to this wave's activation buffers in
// global memory (the L2), each lane storing its four output rows of a tile as one float4 at
// [T][lane]; they are the next layer's B operands of k-quad T as they stand (the input order
// kappa(L, s, g) = 16 (s / 4) + 4 g + s mod 4), so every lane reads back only what it wrote. The
// weights stream from the L2 one quad ahead of their MFMAs. scr: this wave's two buffers of
// wl.maxT * 256 floats (layers alternate between them); hid: LDS scratch for the log-prob terms.
template <int ACT, class LoadT>
__device__ __forceinline__ void policy_tile_wide(const TileArgs& a, const float* qpos, const float* qvel,
                                                 const float* pact, const unsigned* rngc, unsigned long long seed,
                                                 int N, int t, int w, bool valid, float* hid, float* scr, LoadT ld) {
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));
  const WideLayout& L = a.wl;
  float x[kObsSteps];
  tile_observation(a, a.Wt + L.nrm_off, qpos, qvel, pact, N, t, w, valid, lane, ld, x);
  // buffer b of the two (pointer arithmetic on the kernel argument, so that the accesses compile to
  // global loads and stores: a flat access would make every wait count the LDS as well)
  float4* const buf0 = reinterpret_cast<float4*>(scr);
  const long bstride = (long)L.maxT * 64;
  f32x4 hd[kHeadT];
  const float4* W = reinterpret_cast<const float4*>(a.Wt);
  wide_layer<ACT, kWideGroup, true, false>(W + L.woff[0] / 4, a.Wt + L.boff[0], L.nT[0], L.nQ[0], nullptr, x, buf0,
                                           hd, lane);
#pragma unroll 1
  for (int ly = 1; ly < L.nl; ++ly)
    wide_layer<ACT, kWideGroup, false, false>(W + L.woff[ly] / 4, a.Wt + L.boff[ly], L.nT[ly], L.nQ[ly],
                                              buf0 + ((ly - 1) & 1) * bstride, x, buf0 + (ly & 1) * bstride, hd, lane);
  wide_layer<ACT, kHeadT, false, true>(W + L.woff[L.nl] / 4, a.Wt + L.boff[L.nl], kHeadT, L.nQ[L.nl],
                                       buf0 + ((L.nl - 1) & 1) * bstride, x, nullptr, hd, lane);
  tile_outputs(a, hd, a.Wt + L.ls_off, rngc, seed, N, t, w, valid, lane, hid, ld);
}

}  // namespace g1k
