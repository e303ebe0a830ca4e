// tree.h -- ancestor tables of the G1 kinematic tree for forward kinematics by ancestor doubling.
//
// Shared by the GPU kernels and the CPU oracle (plain constexpr C++, no device code). Round r of
// the doubling composes every body's transform with the one held by its 2^r-th ancestor; after
// kFkRounds rounds every body is expressed in the world frame (tree depth < 2^kFkRounds).
#pragma once

#include "g1_model_tables.h"

namespace g1 {

constexpr int kFkRounds = 4;
constexpr int kTreeLanes = 32;   // one entry per lane of a 32-lane world group (lanes >= kNBody: none)

// a[r][b]: the 2^r-th ancestor of body b, or 0 when that would be the world body or lie beyond it
// (then b's transform is already relative to the world, and round r composes it with the world
// body's identity, which leaves it unchanged up to the sign of an exact zero).
struct AncestorTable {
  int a[kFkRounds][kTreeLanes];
};

constexpr AncestorTable make_ancestor_table() {
  AncestorTable t{};
  for (int r = 0; r < kFkRounds; ++r)
    for (int b = 0; b < kTreeLanes; ++b) {
      int x = b < kNBody ? b : 0;
      for (int s = 0; s < (1 << r) && x > 0; ++s) x = body_parent[x];
      t.a[r][b] = x;
    }
  return t;
}

constexpr AncestorTable kAncestors = make_ancestor_table();

// The same table as one 32-bit word per lane, byte r = a[r][b]: one lane-indexed load serves every
// round of the doubling.
struct AncestorWords {
  unsigned w[kTreeLanes];
};

constexpr AncestorWords make_ancestor_words() {
  AncestorWords t{};
  for (int b = 0; b < kTreeLanes; ++b)
    for (int r = 0; r < kFkRounds; ++r) t.w[b] |= (unsigned)kAncestors.a[r][b] << (8 * r);
  return t;
}

constexpr AncestorWords kAncestorWords = make_ancestor_words();
static_assert(kFkRounds <= 4 && kTreeLanes <= 256, "one byte per round in a 32-bit word");

constexpr bool depth_fits_doubling() {
  for (int b = 0; b < kNBody; ++b)
    if (body_depth[b] >= (1 << kFkRounds)) return false;
  return true;
}
static_assert(depth_fits_doubling(), "kFkRounds rounds of doubling reach the world from every body");

}  // namespace g1
