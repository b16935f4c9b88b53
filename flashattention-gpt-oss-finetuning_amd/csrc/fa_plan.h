// fa_plan.h - which key blocks / query rows each workgroup and wave visits.
//
// Shared by the kernels (device) and by the host: fa_capi.cpp sizes the sink split with it, and
// tests/plan_check.cpp compiles this same header with g++ (FA_HOST_ONLY) to check that every
// allowed (query, key) pair is visited exactly once.  W and S are the clamped window and sink
// (0 <= W, S <= L).
//
// Mask (benchmark_backward_speed.py:40-46): allowed(q, k) = k <= q && (q - k < W || k < S).
#pragma once

#ifdef FA_HOST_ONLY
#define FA_HD inline
#else
#include <hip/hip_runtime.h>
#define FA_HD __host__ __device__ __forceinline__
#endif

namespace fa {

constexpr int kLdsKeys = 64;  // keys per LDS block of the query-major kernels
constexpr int kStep = 32;     // keys (or query rows) per MFMA tile edge

FA_HD int imin(int a, int b) { return a < b ? a : b; }
FA_HD int imax(int a, int b) { return a > b ? a : b; }

// dq = q - k.  Bitwise operators (no short-circuit), so the kernels get selects, not branches.
FA_HD bool allowed(int dq, int k, int W, int S) { return (dq >= 0) & ((dq < W) | (k < S)); }

// ---- query-major kernels (forward, dQ) --------------------------------------------------------
// A workgroup owns rows [q0, q0 + bm).  It visits, in LDS blocks of 64 keys, the sink blocks
// [0, min(S, ws)) and then the window blocks [ws, min(q0 + bm, L)), where ws is the first key
// any of its rows can see through the window, rounded down to 64 (the two-phase order of
// benchmark_backward_speed.py:185-208; flash_attention_gpt_oss.py:59-167 has the same idea with
// a separate diagonal phase).  Sink blocks end at or before ws, so no key is visited twice.
struct QPlan {
  int ws, nsb, nb;
};

FA_HD QPlan qplan(int q0, int bm, int L, int W, int S) {
  QPlan p;
  if (q0 >= L) {  // a tile past the end of its sequence (variable-length batches): nothing to visit
    p.ws = 0;
    p.nsb = 0;
    p.nb = 0;
    return p;
  }
  const int q_end = imin(q0 + bm, L);
  p.ws = (imax(0, q0 - W + 1) / kLdsKeys) * kLdsKeys;
  const int sink_end = imin(S, p.ws);
  p.nsb = (sink_end + kLdsKeys - 1) / kLdsKeys;
  p.nb = p.nsb + (q_end - p.ws + kLdsKeys - 1) / kLdsKeys;
  return p;
}

FA_HD int qplan_block(const QPlan& p, int i) { return i < p.nsb ? i * kLdsKeys : p.ws + (i - p.nsb) * kLdsKeys; }

// Does the wave owning rows [qw, qw + 32) need the 32 keys starting at ks0?  (Sinks, or an
// overlap with its own window [qw - W + 1, qw + 31].)
FA_HD bool wave_needs(int ks0, int qw, int L, int W, int S) {
  const int lo = qw - W + 1, hi = imin(qw + 31, L - 1);
  return ks0 < S || (ks0 + 31 >= lo && ks0 <= hi);
}

// Is every pair of rows [qr, qr + 32) x keys [ks0, ks0 + 32) allowed?  (Then the kernels skip
// the per-element mask.  Rows >= L may be included: their results are never stored.)
FA_HD bool tile_full(int ks0, int qr, int W, int S) {
  return (ks0 + 31 <= qr) && ((qr + 31 - ks0 < W) || (ks0 + 32 <= S));
}

// ---- the sliding dQ kernel (fa_bwd_slide.hip) --------------------------------------------------
// A workgroup walks consecutive 32-row tiles; tile m (rows [32m, 32m + 32)) visits the 32-key
// window halves slide_hlo(m, W) .. m (those with wave_needs) and, when slide_sink_half(m, W, S),
// the sink half (keys [0, 32)) before them.  Half j lives in ring slot j % kSlideRing; tile m's
// halves span at most kSlideRing - 1 consecutive indices (W <= kSlideMaxW), so the slot of half
// m + 1, loaded during tile m, is not one that tile m reads.
constexpr int kSlideRing = 7;
constexpr int kSlideMaxW = 32 * (kSlideRing - 2) + 1;  // 161
// The sliding forward (fa_fwd.hip fwd_slide_kernel) keeps two workgroups per CU, so its ring is
// one slot shorter: W <= 129.
constexpr int kFwdSlideRing = 6;
constexpr int kFwdSlideMaxW = 32 * (kFwdSlideRing - 2) + 1;  // 129

// First window half of tile m: the half holding key 32m - W + 1 (clamped to 0); W >= 1.
FA_HD int slide_hlo(int m, int W) {
  const int back = (W - 1 + 31) / 32;  // ceil((W - 1) / 32)
  return m > back ? m - back : 0;
}

// Does tile m visit the sink half separately (it holds sink keys and is not a window half)?
FA_HD bool slide_sink_half(int m, int W, int S) { return S > 0 && slide_hlo(m, W) > 0; }

// ---- key-major kernel (dK, dV) ----------------------------------------------------------------
// A workgroup owns the kKvKeys keys [kKvKeys*kblk, +kKvKeys); each of its waves owns a 32-key
// half.  The rows that can see a 32-key half [ks0, ks0 + 32) through the window are
// [ks0, ks0 + 31 + W); the workgroup sweeps the union of its halves' ranges,
// [kKvKeys*kblk, kv_window_end), each wave from its own first key on (a half's sink keys are
// also seen by the rows between its own window end and the workgroup's).  For the first `nsp`
// blocks (those holding sink keys with rows beyond kv_window_end) the remaining rows
// [kv_window_end, L) only see the sink keys; they are split into chunks of chunk_rows handled by
// extra workgroups.  Chunks are laid out from the window end rounded down to 32 rows (so a
// chunk covers whole 32-row blocks): chunk c covers [max(base + c*chunk_rows, end),
// min(base + (c+1)*chunk_rows, L)), base = end rounded down to a multiple of 32.
constexpr int kKvKeys = 64;

FA_HD int kv_rows_end(int ks0, int nkeys, int L, int W) { return imin(L, ks0 + nkeys - 1 + W); }

FA_HD int kv_window_end(int kblk, int L, int W) { return kv_rows_end(kKvKeys * kblk, kKvKeys, L, W); }

// Does the wave owning keys [ks0, ks0 + 32) have any allowed pair with rows [qr0, qr0 + 32)?
// Rows past the half's window only see its sink keys.
FA_HD bool kv_half_needs(int qr0, int ks0, int L, int W, int S) {
  return qr0 + 31 >= ks0 && (ks0 < S || qr0 < kv_rows_end(ks0, 32, L, W));
}

FA_HD int kv_chunk_base(int kblk, int L, int W) { return kv_window_end(kblk, L, W) / 32 * 32; }

FA_HD int kv_chunk_lo(int kblk, int c, int chunk_rows, int L, int W) {
  return imax(kv_chunk_base(kblk, L, W) + c * chunk_rows, kv_window_end(kblk, L, W));
}

FA_HD int kv_chunk_hi(int kblk, int c, int chunk_rows, int L, int W) {
  return imin(kv_chunk_base(kblk, L, W) + (c + 1) * chunk_rows, L);
}

// Number of leading key blocks whose sink rows are chunked: blocks holding a key < S whose
// window end is before L.  (Both conditions hold on a prefix of the blocks.)
FA_HD int kv_sink_blocks(int L, int W, int S) {
  int n = 0;
  for (int kb = 0; kKvKeys * kb < S; ++kb)
    if (kv_window_end(kb, L, W) < L) n = kb + 1;
  return n;
}

// Chunks per chunked block: enough for block 0, whose window ends first.
FA_HD int kv_n_chunks(int L, int W, int S, int chunk_rows) {
  return kv_sink_blocks(L, W, S) > 0 ? (L - kv_chunk_base(0, L, W) + chunk_rows - 1) / chunk_rows : 0;
}

// ---- sink rows in the dQ kernel ------------------------------------------------------------------
// With at most kDqSinkKeys sink keys (all in key block 0) and rows past block 0's window, the dQ
// kernel -- which visits keys [0, 32) for every query tile -- also accumulates the sink keys' dK/dV
// contributions of those rows, [dq_sink_row0, L); the key-major kernel then runs no chunk
// workgroups and covers only rows [0, dq_sink_row0) of block 0.
constexpr int kDqSinkKeys = 16;

FA_HD bool dq_sink_mode(int L, int W, int S) { return S >= 1 && S <= kDqSinkKeys && kv_sink_blocks(L, W, S) == 1; }

FA_HD int dq_sink_row0(int L, int W) { return kv_window_end(0, L, W); }

// ---- key-major kernel with 32-key workgroups (bwd_dkdv4_kernel) ---------------------------------
// A workgroup owns the 32 keys [ks0, ks0 + 32) and its 4 waves take 4 query heads at a time, each
// staging its own (head, 32-row block) items, so every wave needs the same row blocks.  It sweeps
// rows [ks0, kv4_rows_end): the window's rows, and for a half holding sink keys every later row
// (up to dq_sink_row0 in dq_sink_mode, where the dQ kernel takes the rest).  It serves only shapes
// without chunked sink rows (nsp == 0, or dq_sink_mode).
FA_HD int kv4_rows_end(int ks0, int L, int W, int S, bool dq_sink) {
  if (ks0 < S) return dq_sink ? dq_sink_row0(L, W) : L;
  return kv_rows_end(ks0, 32, L, W);
}

}  // namespace fa
