// plan_check.cpp - host check of the kernels' visit plan (csrc/fa_plan.h compiled with g++).
//
// Walks the loops of the query-major kernels (fa_fwd.hip fwd_kernel, fa_bwd.hip bwd_dq_kernel,
// fa_bwd_slide.hip bwd_dq_slide_kernel) and of the key-major kernels (bwd_dkdv_kernel,
// bwd_dkdv4_kernel) over many (L, W, S, rows-per-workgroup, chunk size) cases and checks that
//   * every allowed (q, k) pair is visited exactly once and no other pair is counted,
//   * a tile reported "full" (mask skipped) holds only allowed pairs,
//   * the key-major row ranges of the regular and chunk workgroups partition the rows that can
//     see each key block.
// Prints "OK <cases>" or the first failing case; exit status 0 on success.
#define FA_HOST_ONLY 1
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../flashattention-gpt-oss-finetuning_amd/csrc/fa_plan.h"

using namespace fa;

static bool ref_allowed(int q, int k, int W, int S) { return k <= q && (q - k < W || k < S); }

static int fail(const char* what, int L, int W, int S, int x, int q, int k, int got) {
  std::printf("FAIL %s L=%d W=%d S=%d param=%d q=%d k=%d count=%d\n", what, L, W, S, x, q, k, got);
  return 1;
}

// Query-major: workgroups of bm = 32*wq rows, waves of 32 rows.
static int check_qmajor(int L, int W, int S, int wq) {
  const int bm = 32 * wq;
  std::vector<int> cnt(size_t(L) * L, 0);
  for (int q0 = 0; q0 < L; q0 += bm) {
    const QPlan p = qplan(q0, bm, L, W, S);
    for (int i = 0; i < p.nb; ++i) {
      const int kb = qplan_block(p, i);
      if (kb < 0 || kb >= L) return fail("block out of range", L, W, S, wq, q0, kb, 0);
      for (int w = 0; w < wq; ++w) {
        const int qw = q0 + 32 * w;
        if (qw >= L) continue;  // the kernel skips inactive waves
        for (int sb = 0; sb < 2; ++sb) {
          const int ks0 = kb + 32 * sb;
          if (!wave_needs(ks0, qw, L, W, S)) continue;
          const bool full = tile_full(ks0, qw, W, S);
          for (int r = 0; r < 32; ++r)
            for (int c = 0; c < 32; ++c) {
              const int q = qw + r, k = ks0 + c;
              if (q >= L) continue;  // rows >= L are never stored
              const bool ok = full || allowed(q - k, k, W, S);
              if (full && !(k < L && ref_allowed(q, k, W, S))) return fail("full tile has a masked pair", L, W, S, wq, q, k, 0);
              if (ok && k < L) ++cnt[size_t(q) * L + k];
              if (ok && k >= L) return fail("key beyond L passes the mask", L, W, S, wq, q, k, 0);
            }
        }
      }
    }
  }
  for (int q = 0; q < L; ++q)
    for (int k = 0; k < L; ++k) {
      const int want = ref_allowed(q, k, W, S) ? 1 : 0;
      if (cnt[size_t(q) * L + k] != want) return fail("q-major visit count", L, W, S, wq, q, k, cnt[size_t(q) * L + k]);
    }
  return 0;
}

// The sliding dQ kernel and forward (1 <= W <= kSlideMaxW, resp. kFwdSlideMaxW; S <= 32): 32-row
// tiles, each visiting the sink half
// (when slide_sink_half) and then the window halves slide_hlo .. m that wave_needs.  Also checks
// that a tile's halves span at most kSlideRing - 1 indices (the ring slot of half m + 1 is free
// during tile m) and that, in dq_sink_mode, every tile with rows past dq_sink_row0 visits the sink
// half (where the kernel accumulates the sink keys' dK/dV).
static int check_slide(int L, int W, int S) {
  std::vector<int> cnt(size_t(L) * L, 0);
  for (int m = 0; 32 * m < L; ++m) {
    const int qw = 32 * m, hlo = slide_hlo(m, W);
    if (m - hlo > kSlideRing - 2) return fail("slide window spans too many halves", L, W, S, m, qw, hlo, 0);
    if (W <= kFwdSlideMaxW && m - hlo > kFwdSlideRing - 2)
      return fail("forward slide window spans too many halves", L, W, S, m, qw, hlo, 0);
    if (dq_sink_mode(L, W, S) && qw + 31 >= dq_sink_row0(L, W) && !slide_sink_half(m, W, S))
      return fail("slide sink rows without the sink half", L, W, S, m, qw, 0, 0);
    auto visit = [&](int ks0) {
      const bool full = tile_full(ks0, qw, W, S);
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          const int q = qw + r, k = ks0 + c;
          if (q >= L) continue;
          const bool ok = full || allowed(q - k, k, W, S);
          if (full && !(k < L && ref_allowed(q, k, W, S))) return fail("slide full half has a masked pair", L, W, S, m, q, k, 0);
          if (ok && k >= L) return fail("slide key beyond L passes the mask", L, W, S, m, q, k, 0);
          if (ok) ++cnt[size_t(q) * L + k];
        }
      return 0;
    };
    if (slide_sink_half(m, W, S) && visit(0)) return 1;
    for (int j = hlo; j <= m; ++j)
      if (wave_needs(32 * j, qw, L, W, S) && visit(32 * j)) return 1;
  }
  for (int q = 0; q < L; ++q)
    for (int k = 0; k < L; ++k) {
      const int want = ref_allowed(q, k, W, S) ? 1 : 0;
      if (cnt[size_t(q) * L + k] != want) return fail("slide visit count", L, W, S, 0, q, k, cnt[size_t(q) * L + k]);
    }
  return 0;
}

// In dq_sink_mode, the dQ kernel's sink rows: every query tile of wq 32-row waves visits keys
// [0, 32) through its plan; rows >= dq_sink_row0 add keys [0, kDqSinkKeys) where allowed, keys < S
// counted.
static int count_dq_sink_rows(std::vector<int>& cnt, int L, int W, int S) {
  if (S > kDqSinkKeys) return fail("dq sink mode with too many sink keys", L, W, S, 0, 0, 0, S);
  const int row0 = dq_sink_row0(L, W);
  for (int wq : {1, 2, 4})
    for (int q0 = 0; q0 < L; q0 += 32 * wq) {
      const QPlan p = qplan(q0, 32 * wq, L, W, S);
      const bool visits0 = p.nb > 0 && qplan_block(p, 0) == 0;
      for (int w = 0; w < wq; ++w) {
        const int qw = q0 + 32 * w;
        if (qw >= L || qw + 31 < row0) continue;
        if (!visits0 || !wave_needs(0, qw, L, W, S)) return fail("dq sink tile misses key block 0", L, W, S, wq, qw, 0, 0);
        if (wq != 1) continue;  // count once
        for (int q = qw; q < qw + 32 && q < L; ++q)
          for (int k = 0; k < S; ++k)
            if (q >= row0 && allowed(q - k, k, W, S)) ++cnt[size_t(q) * L + k];
      }
    }
  return 0;
}

// Key-major: regular workgroups per kKvKeys-key block (waves per 32-key half), plus chunk
// workgroups for the sink blocks.  A wave sweeps the workgroup's rows from its own first key on,
// skipping q-blocks that kv_half_needs rules out, and, in a chunk workgroup, halves without sink
// keys.
static int check_kvmajor(int L, int W, int S, int chunk_rows) {
  std::vector<int> cnt(size_t(L) * L, 0);
  const int nkb = (L + kKvKeys - 1) / kKvKeys;
  const int nsp = kv_sink_blocks(L, W, S);
  const int n_chunks = kv_n_chunks(L, W, S, chunk_rows);
  auto sweep = [&](int kblk, int qlo, int qhi, bool chunk) -> int {
    if (qhi <= qlo) return 0;
    for (int qb = qlo / 32; qb < (qhi + 31) / 32; ++qb) {
      const int qr0 = 32 * qb;
      for (int kh = 0; kh < kKvKeys / 32; ++kh) {
        const int ks0 = kKvKeys * kblk + 32 * kh;
        if (ks0 >= L) continue;
        if (chunk && ks0 >= S) continue;
        const int hqlo = chunk ? qlo : imax(qlo, ks0);
        const int hqhi = qhi;
        if (qr0 + 32 <= hqlo || qr0 >= hqhi) continue;  // q-block outside this half's rows
        if (!kv_half_needs(qr0, ks0, L, W, S)) continue;  // beyond the half's window, no sinks
        const bool full = (qr0 >= hqlo) && (qr0 + 32 <= hqhi) && tile_full(ks0, qr0, W, S);
        for (int r = 0; r < 32; ++r)
          for (int c = 0; c < 32; ++c) {
            const int q = qr0 + r, k = ks0 + c;
            const bool ok = full || (q >= hqlo && q < hqhi && allowed(q - k, k, W, S));
            if (!ok) continue;
            if (q >= L || k >= L) {
              if (full) return fail("full kv tile beyond L", L, W, S, chunk_rows, q, k, 0);
              return fail("kv pair beyond L passes", L, W, S, chunk_rows, q, k, 0);
            }
            if (full && !ref_allowed(q, k, W, S)) return fail("full kv tile has a masked pair", L, W, S, chunk_rows, q, k, 0);
            ++cnt[size_t(q) * L + k];
          }
      }
    }
    return 0;
  };
  for (int kblk = 0; kblk < nkb; ++kblk)
    if (sweep(kblk, kKvKeys * kblk, kv_window_end(kblk, L, W), false)) return 1;
  if (dq_sink_mode(L, W, S)) {
    if (nsp != 1) return fail("dq sink mode with too many sink keys", L, W, S, chunk_rows, 0, 0, nsp);
    if (count_dq_sink_rows(cnt, L, W, S)) return 1;
  } else {
    for (int kblk = 0; kblk < nsp; ++kblk)
      for (int c = 0; c < n_chunks; ++c)
        if (sweep(kblk, kv_chunk_lo(kblk, c, chunk_rows, L, W), kv_chunk_hi(kblk, c, chunk_rows, L, W), true)) return 1;
  }
  for (int q = 0; q < L; ++q)
    for (int k = 0; k < L; ++k) {
      const int want = ref_allowed(q, k, W, S) ? 1 : 0;
      if (cnt[size_t(q) * L + k] != want) return fail("kv-major visit count", L, W, S, chunk_rows, q, k, cnt[size_t(q) * L + k]);
    }
  return 0;
}

// Key-major with 32-key workgroups (fa_bwd.hip bwd_dkdv4_kernel; shapes with nsp == 0 or in
// dq_sink_mode): keys [ks0, ks0 + 32) sweep the 32-row blocks of [ks0, kv4_rows_end) that
// kv_half_needs keeps, with the kernel's own mask: key k passes row q when 0 <= q - k < lim(k),
// lim = W for window keys, rows_end - k for sink keys whose later rows the dQ kernel takes, and
// unbounded for other sink keys.  Pairs with q >= L or k >= L may pass the mask: their Q rows and
// K rows are zero-filled and their dK/dV rows are never stored, so only pairs inside L are counted.
static int check_kv4(int L, int W, int S) {
  const bool dqs = dq_sink_mode(L, W, S);
  if (!(kv_sink_blocks(L, W, S) == 0 || dqs)) return 0;  // not served by this kernel
  std::vector<int> cnt(size_t(L) * L, 0);
  for (int ks0 = 0; ks0 < L; ks0 += 32) {
    const int qlo = ks0, qhi = kv4_rows_end(ks0, L, W, S, dqs);
    if (qhi <= qlo) continue;
    for (int qb = qlo / 32; qb < (qhi + 31) / 32; ++qb) {
      const int qr0 = 32 * qb;
      if (!kv_half_needs(qr0, ks0, L, W, S)) continue;
      const bool full = qr0 + 32 <= qhi && tile_full(ks0, qr0, W, S);
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          const int q = qr0 + r, k = ks0 + c;
          const long lim = k < S ? (dqs ? long(imax(qhi - k, 0)) : 0x80000000L) : long(W);
          const bool ok = full || (q - k >= 0 && long(q - k) < lim);
          if (!ok) continue;
          if (full && (q >= L || k >= L || !ref_allowed(q, k, W, S)))
            return fail("full kv4 tile has a masked pair", L, W, S, 32, q, k, 0);
          if (q >= L || k >= L) continue;
          ++cnt[size_t(q) * L + k];
        }
    }
  }
  if (dqs && count_dq_sink_rows(cnt, L, W, S)) return 1;
  for (int q = 0; q < L; ++q)
    for (int k = 0; k < L; ++k) {
      const int want = ref_allowed(q, k, W, S) ? 1 : 0;
      if (cnt[size_t(q) * L + k] != want) return fail("kv4 visit count", L, W, S, 32, q, k, cnt[size_t(q) * L + k]);
    }
  return 0;
}

int main() {
  const int Ls[] = {1, 2, 5, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 200, 257, 300, 513};
  const int Ws[] = {0, 1, 2, 5, 31, 32, 33, 64, 100, 128, 129, 160, 161, 162, 256, 100000};
  const int Ss[] = {0, 1, 4, 16, 31, 32, 33, 64, 65, 100, 100000};
  long cases = 0;
  for (int L : Ls)
    for (int Wr : Ws)
      for (int Sr : Ss) {
        if (Wr < 1 && Sr < 1) continue;  // rejected by the C ABI
        const int W = Wr > L ? L : Wr, S = Sr > L ? L : Sr;  // clamped as in fa_capi.cpp
        for (int wq : {1, 2, 4}) {
          if (check_qmajor(L, W, S, wq)) return 1;
          ++cases;
        }
        for (int cr : {32, 64, 256}) {
          if (check_kvmajor(L, W, S, cr)) return 1;
          ++cases;
        }
        if (W >= 1 && W <= 512) {
          if (check_kv4(L, W, S)) return 1;
          ++cases;
        }
        if (W >= 1 && W <= kSlideMaxW && S <= 32) {
          if (check_slide(L, W, S)) return 1;
          ++cases;
        }
      }
  std::printf("OK %ld\n", cases);
  return 0;
}
