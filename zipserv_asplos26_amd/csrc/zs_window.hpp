// zs_window.hpp -- exponent-window selection on the GPU (both rules), as
// wave-level routines over a 256-bin histogram, shared by the selection
// kernels of zs_encode.hip and the one-pass re-tiled encoder's window check.
#pragma once
#include "zs_device.hpp"

namespace zs {

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Shared tail of both window rules (kernel_benchmark/utils.h:228-270,
// zipserv_decode_attention_ext.cu:103-133): the 7 candidates (exponents;
// missing ones already filled with 127 - i), sorted; the first candidate
// whose 7-exponent window has only positive counts wins, else the start of
// the longest run of consecutive candidates (clamped to [0, 248] by the GPU
// rule only).  Every array index is a compile-time constant, so the
// candidates stay in registers (a dynamic index would put them in scratch
// memory, one memory round trip per access).
__device__ __forceinline__ void window_from_candidates(const int64_t* counts, int (&cand)[7],
                                                       bool clamp, int32_t* top,
                                                       const int32_t* guess, int32_t* differs) {
#pragma unroll
  for (int i = 0; i < 6; ++i)  // bubble sort; ties are equal values, so any sort agrees
#pragma unroll
    for (int j = 0; j < 6 - i; ++j) {
      const int lo = min(cand[j], cand[j + 1]), hi = max(cand[j], cand[j + 1]);
      cand[j] = lo;
      cand[j + 1] = hi;
    }
  int win = -1;
#pragma unroll
  for (int c = 0; c < 7; ++c) {
    const int st = cand[c];
    if (win < 0 && st >= 0 && st + 6 <= 255) {
      bool all = true;
      for (int i = 0; i < 7; ++i) all = all && counts[st + i] > 0;
      if (all) win = st;
    }
  }
  if (win < 0) {
    int best = cand[0], best_len = 1, run = 1;
#pragma unroll
    for (int i = 1; i < 7; ++i) {
      run = (cand[i] == cand[i - 1] + 1) ? run + 1 : 1;
      if (run > best_len) {
        best_len = run;
        best = cand[i] - run + 1;
      }
    }
    win = clamp ? (best < 0 ? 0 : (best > 248 ? 248 : best)) : best;
  }
#pragma unroll
  for (int i = 0; i < 7; ++i) top[i] = win + i;
  if (guess) *differs = guess[0] != win;  // windows are 7 consecutive exponents
}

// Seven wave-wide maxima of key = (count << 8 | 255 - exponent) over the
// exponents not taken yet (lane i holds exponents i, i + 64, i + 128,
// i + 192; zero counts have key 0 and are never taken): cand[t] is the
// exponent of pass t, or 127 - t once no positive count is left.  Returns the
// number of exponents taken; *c7 is the count of the last one taken.
__device__ __forceinline__ int top7_passes(int64_t (&key)[4], int l, int (&cand)[7],
                                           int64_t* c7) {
  int taken = 0;
#pragma unroll
  for (int t = 0; t < 7; ++t) {
    int64_t best = key[0];
#pragma unroll
    for (int k = 1; k < 4; ++k) best = key[k] > best ? key[k] : best;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int64_t o = __shfl_xor(best, off);
      best = o > best ? o : best;
    }
    const int e = 255 - (int)(best & 0xFF);
    cand[t] = best == 0 ? 127 - t : e;
    if (best != 0) {
      ++taken;
      *c7 = best >> 8;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (best != 0 && 64 * k + l == e) key[k] = 0;
  }
  return taken;
}

// Window selection of zipserv_decode_attention_ext.cu:65-134: seven slots
// start at count -1 (so zero counts can be taken); each exponent 0..255
// replaces the first minimum slot on strictly greater count; candidates are
// sorted, the first one starting 7 present exponents wins, else the start of
// the longest consecutive run, clamped to [0, 248].  Run by one whole wave
// (l = lane) over counts[256] (the caller's LDS); lane 0 writes top[0..6]
// and, with a guess, *differs.  The streaming top-7 runs on wave-uniform
// values (scalar unit), reading each count with v_readlane instead of a
// dependent memory load.
__device__ __forceinline__ void select_kv_wave(const int64_t* counts, int l, int32_t* top,
                                               const int32_t* guess, int32_t* differs) {
  int64_t cv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) cv[k] = counts[64 * k + l];
  // When exactly seven exponents have a count >= the seventh largest count
  // c7 > 0, those seven are the final slots whatever the order: one of them
  // is rejected or evicted only while seven others with counts >= its own
  // sit in the slots, which would make eight.  Only then is the streaming
  // walk below skipped.
  {
    int64_t key[4], c7 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) key[k] = cv[k] > 0 ? (cv[k] << 8) | (255 - (64 * k + l)) : 0;
    int cand[7];
    if (top7_passes(key, l, cand, &c7) == 7) {
      int ge = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) ge += __builtin_popcountll(__builtin_amdgcn_ballot_w64(cv[k] >= c7));
      if (ge == 7) {
        if (l == 0) window_from_candidates(counts, cand, true, top, guess, differs);
        return;
      }
    }
  }
  int te[7];
  int64_t tc[7];
#pragma unroll
  for (int i = 0; i < 7; ++i) {
    te[i] = -1;
    tc[i] = -1;
  }
  // Only an exponent whose count beats the current minimum slot changes the
  // slots, and the minimum never decreases: walk just those (a ballot of
  // count > min, refreshed after every change), in exponent order.  The
  // first minimum slot is replaced; its count is the running minimum tmin,
  // so the slot is found by comparing against tmin (no dynamic index).
  int64_t tmin = -1;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint64_t mask = __builtin_amdgcn_ballot_w64(cv[k] > tmin);
    while (mask) {
      const int j = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int64_t c = readlane64(cv[k], j);
      if (c > tmin) {
        bool done = false;
#pragma unroll
        for (int i = 0; i < 7; ++i)
          if (!done && tc[i] == tmin) {
            tc[i] = c;
            te[i] = 64 * k + j;
            done = true;
          }
        tmin = tc[0];
#pragma unroll
        for (int i = 1; i < 7; ++i) tmin = tc[i] < tmin ? tc[i] : tmin;
        mask &= __builtin_amdgcn_ballot_w64(cv[k] > tmin);
      }
    }
  }
  if (l != 0) return;
  // Slots fill in index order, so untaken slots (-1) form a suffix: slot i
  // untaken is candidate i missing, filled with 127 - i.
  int cand[7];
#pragma unroll
  for (int i = 0; i < 7; ++i) cand[i] = te[i] >= 0 ? te[i] : 127 - i;
  window_from_candidates(counts, cand, true, top, guess, differs);
}

// Window selection of kernel_benchmark/utils.h:189-272 (the host analyzer of
// the weights path) on the device: seven passes each take the strictly
// largest count not taken yet -- ties go to the lowest exponent and zero
// counts are never taken -- missing candidates are filled with 127 - n, and
// the tail is select_kv_wave's without the [0, 248] clamp.  One wave; lane i
// holds exponents i, i + 64, i + 128, i + 192; a pass is one wave-wide
// maximum of (count << 8 | 255 - exponent) over the exponents not taken.
__device__ __forceinline__ void select_weights_wave(const int64_t* counts, int l, int32_t* top,
                                                    const int32_t* guess, int32_t* differs) {
  int64_t key[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t c = counts[64 * k + l];
    // counts stay below 2^55 (numel < 2^63 / 256 is far past any tensor)
    key[k] = c > 0 ? (c << 8) | (255 - (64 * k + l)) : 0;
  }
  int cand[7];
  int64_t c7;
  top7_passes(key, l, cand, &c7);
  if (l != 0) return;
  window_from_candidates(counts, cand, false, top, guess, differs);
}

__device__ __forceinline__ void select_window_wave(bool weights_rule, const int64_t* counts, int l,
                                                   int32_t* top, const int32_t* guess,
                                                   int32_t* differs) {
  if (weights_rule)
    select_weights_wave(counts, l, top, guess, differs);
  else
    select_kv_wave(counts, l, top, guess, differs);
}

}  // namespace zs
