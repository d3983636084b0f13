// Shared pieces of the strong-hierarchy (HType.STRONG) Mamba-2 kernels: the
// strong level function of base.py:49-62 evaluated at compile time, its two
// 64 x 64 chunk tables and, for the backward's dlambda, the source range of
// every (target position, level) pair.
#pragma once

#include "mamba2_common.h"

namespace hattn {

constexpr int kSC = 64;           // chunk
constexpr int kSMaxLev = 10;      // chunk-level levels 0 .. 9 (T <= 64 * 2^9)
constexpr int kSLocLev = 8;       // levels of the diagonal / sub-diagonal blocks (0 .. 7)

struct alignas(16) StrongTables {
  unsigned char intra[kSC * kSC];   // [a][b], a >= b: level of (a, b) inside a chunk
  unsigned char sub[kSC * kSC];     // [a][b]: level of (64 + a, b)
  constexpr StrongTables() : intra(), sub() {
    for (int a = 0; a < kSC; ++a)
      for (int b = 0; b < kSC; ++b) {
        intra[a * kSC + b] = (unsigned char)(b < a ? strong_level_ce(a, b) : 0);
        sub[a * kSC + b] = (unsigned char)strong_level_ce(kSC + a, b);
      }
  }
};

// For target position a of a chunk, its sources in the order "previous chunk
// b = 0 .. 63, then this chunk b = 0 .. a" (index i = b, resp. 64 + b).  The
// strong level is non-increasing along that order (each level of the
// recurrent state holds one contiguous run of tokens, older runs on higher
// levels), so the sources of level l form the index range [lo, hi); an absent
// level has lo == hi.
struct StrongRanges {
  unsigned char lo[kSC][kSLocLev], hi[kSC][kSLocLev];
  constexpr StrongRanges() : lo(), hi() {
    for (int a = 0; a < kSC; ++a) {
      for (int l = 0; l < kSLocLev; ++l) {
        lo[a][l] = 0;
        hi[a][l] = 0;
      }
      bool seen[kSLocLev] = {};
      for (int i = 0; i <= kSC + a; ++i) {
        const int b = i < kSC ? i : i - kSC;
        const int l = i < kSC ? strong_level_ce(kSC + a, b) : (b < a ? strong_level_ce(a, b) : 0);
        if (!seen[l]) {
          lo[a][l] = (unsigned char)i;
          seen[l] = true;
        }
        hi[a][l] = (unsigned char)(i + 1);
      }
    }
  }
};

}  // namespace hattn
