// fa_fwd.hip - forward pass: O = softmax(mask(Q K^T * scale)) V and the row log-sum-exp.
//
// Replaces _flash_attention_forward_swa_kernel (flash_attention_gpt_oss.py:7-180) and the
// benchmark's _forward_kernel (benchmark_backward_speed.py:146-217).  Same mathematics (FA-2
// online softmax in the log2 domain), a different decomposition:
//
//  * A tile is 32*wq query rows of HPW*wh query heads of ONE KV group, so every K/V block
//    staged in LDS serves all of those heads.  The grid is one resident wave of 4-wave
//    workgroups; every XCD owns a contiguous range of tiles (neighbouring tiles share K/V rows in
//    its L2) and its workgroups walk it, each loading its next tile's Q rows by LDS DMA while the
//    current tile computes.
//  * Each wave owns 32 query rows x HPW heads and computes the transposed score tile
//    S^T = K Q^T (keys x queries) on v_mfma_f32_32x32x16: the lane that holds column q of S^T
//    owns query row q, so the row max / row sum / rescale of the online softmax are per-lane
//    scalars and only one cross-half exchange is needed per 32-key step.
//  * O^T = V^T P^T accumulates in registers; P^T goes from the C layout of S^T straight into
//    the B operand (see fa_common.h), V^T is staged in LDS in the matching permuted order.
//  * Key blocks are enumerated as in the reference: the sink blocks [0, min(S, ws)) and then the
//    window blocks [ws, q_end) (ws = window start rounded down to the 64-key LDS block), and
//    each wave additionally skips 32-key halves outside its own rows' window.  Tiles that are
//    fully inside the mask skip the per-element mask.
#include "fa_args.h"
#include "fa_common.h"

namespace fa {

constexpr float kRescaleGap = 8.f;  // log2 units: P stays <= 256 between rescales

// Additive masks of the partially masked halves that recur on every tile, built once per
// workgroup in LDS (fwd_patterns): lane l's 16 values at [(e / 4) * 64 + l] * 4 + e % 4 of pattern
// p = 0 (the diagonal half, qw - ks0 = 0), 1 and 2 (the window-edge halves, qw - ks0 = e1 and
// e1 + 32, both multiples of 32 in [W - 31, W + 30]) and 3 (keys [0, 32) seen only as sinks).
constexpr int kPatterns = 4;
constexpr int kPatternFloats = 16 * 64;

struct EdgeOffsets {
  int e1, e2;  // qw - ks0 of the window-edge halves, -1 where there is none
};

__device__ __forceinline__ EdgeOffsets edge_offsets(int W) {
  EdgeOffsets r{-1, -1};
  if (W > 31) {
    r.e1 = (W - 31 + 31) / 32 * 32;
    r.e2 = r.e1 + 32 <= W + 30 ? r.e1 + 32 : -1;
  }
  return r;
}

// Wave p of the workgroup writes pattern p (call with 4 waves, before the first barrier).
__device__ __forceinline__ void fwd_patterns(float* pat, int W, int S) {
  const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
  const int r32 = lane & 31, hf = lane >> 5;
  const EdgeOffsets eo = edge_offsets(W);
  const int dl = p == 1 ? eo.e1 : p == 2 ? eo.e2 : 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int off = 8 * (e / 4) + (e % 4);
    const int d = r32 - 4 * hf - off;  // q - k on the diagonal half
    const bool ok = p == 3 ? 4 * hf + off < S : unsigned(d + dl) < unsigned(W);
    pat[p * kPatternFloats + ((e >> 2) * 64 + lane) * 4 + (e & 3)] = ok ? 0.f : kNegInf;
  }
}

// Q fragments per head and lane: 16 bytes each, head-dim slice [hf*D/2 + 8ks, +8) for 16-bit
// inputs; for e4m3 inputs, fragment f holds bytes [64 (f / 2) + 32 hf + 16 (f % 2), +16) of the
// row, the operand layout of the fp8 MFMA.
// F8 = 0: 16-bit inputs; 1: e4m3 inputs, Q K^T on the fp8 MFMA; 2: also P V on the fp8 MFMA.
template <int D, int F8>
constexpr int kQFrags = F8 ? D / 32 : D / 16;

// Masked scores S^T = K Q^T of one 32-key half [ks0, ks0 + 32) -- the swizzled K tile at Kl --
// for the HPW heads of a wave whose 32 rows start at qw (this lane's row q).
template <typename E, int D, int HPW, int F8>
__device__ __forceinline__ void half_scores(const Args& a, const uint16_t* Kl, int ks0, int qw, int q,
                                            const u32x4 (&qf)[HPW][kQFrags<D, F8>], const float* pat,
                                            EdgeOffsets eo, f32x16 (&s)[HPW]) {
  constexpr int KS = kQFrags<D, F8>;
  const int lane = threadIdx.x & 63;
  const int r32 = lane & 31, hf = lane >> 5;
  const int W = a.W, S = a.S;
  // S^T = K Q^T for every head of the wave (the K fragments are shared).  Masked tiles start
  // the accumulator from an additive bias, 0 (allowed) or -inf (masked), shared by the
  // heads.  Register e of this lane holds key ks0 + 4hf + off(e), off(e) = 8(e/4) + e%4,
  // of row q; with dq0 = q - ks0 - 4hf the test is one unsigned compare,
  // allowed = (dq0 - off) < lim, lim = W for ordinary keys and 2^31 for sink keys (any
  // q >= k).  Which form applies is wave-uniform.
  // Head by head: head 0's scores are complete while head 1's MFMAs are still in the
  // pipe, and head 0's softmax (VALU) overlaps them.
  u32x4 kf[KS];
  if constexpr (F8) {
    // e4m3 K rows of D bytes, swizzled like 16-bit rows of D / 2 elements
#pragma unroll
    for (int f = 0; f < KS; ++f)
      kf[f] = *reinterpret_cast<const u32x4*>(Kl + swz_off<D / 2>(r32, 8 * (4 * (f / 2) + 2 * hf + f % 2)));
  } else {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kf[ks] = *reinterpret_cast<const u32x4*>(Kl + swz_off<D>(r32, hf * (D / 2) + 8 * ks));
  }
  auto qk = [&](const f32x16& c0) {
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      if constexpr (F8) {
#pragma unroll
        for (int kb = 0; kb < KS / 2; ++kb)
          s[h] = mfma_fp8(kf[2 * kb], kf[2 * kb + 1], qf[h][2 * kb], qf[h][2 * kb + 1], kb == 0 ? c0 : s[h]);
      } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s[h] = E::mfma(kf[ks], qf[h][ks], ks == 0 ? c0 : s[h]);
      }
    }
  };
  if (tile_full(ks0, qw, W, S)) {
    qk(f32x16{});
  } else {
    f32x16 bias;
    const int dl = qw - ks0;
    const int pi = ks0 >= S ? (dl == 0 ? 0 : dl == eo.e1 ? 1 : dl == eo.e2 ? 2 : -1)
                            : (ks0 == 0 && S < 32 && qw - 31 >= W ? 3 : -1);
    const int dq0 = q - ks0 - 4 * hf;
    if (pi >= 0) {  // a recurring pattern: four 16-byte LDS reads
      const f32x4* p4 = reinterpret_cast<const f32x4*>(pat + pi * kPatternFloats) + lane;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v = p4[64 * j];
#pragma unroll
        for (int i = 0; i < 4; ++i) bias[4 * j + i] = v[i];
      }
    } else if (ks0 >= S || ks0 + 32 <= S) {  // one limit for all 32 keys
      const unsigned lim = ks0 >= S ? unsigned(W) : 0x80000000u;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        bias[e] = unsigned(dq0 - (8 * (e / 4) + (e % 4))) < lim ? 0.f : kNegInf;
    } else {  // the sink boundary S falls inside these keys
      const int sl = S - ks0 - 4 * hf;  // keys with off < sl are sinks
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int off = 8 * (e / 4) + (e % 4);
        bias[e] = unsigned(dq0 - off) < (off < sl ? 0x80000000u : unsigned(W)) ? 0.f : kNegInf;
      }
    }
    qk(bias);
  }
}

// One 32-key half of the 16-bit P V path: masked scores, the online-softmax update of (m2, lsum,
// acc) and O^T += V^T P^T, V^T read transposed from the swizzled [32][D] 16-bit V tile at Vl.
template <typename E, int D, int HPW, int F8>
__device__ __forceinline__ void fwd_half(const Args& a, const uint16_t* Kl, const uint16_t* Vl, int ks0, int qw, int q,
                                         const u32x4 (&qf)[HPW][kQFrags<D, F8>], float (&m2)[HPW], float (&lsum)[HPW],
                                         f32x16 (&acc)[HPW][D >= 32 ? D / 32 : 1], const float* pat,
                                         EdgeOffsets eo) {
  constexpr int DB = D >= 32 ? D / 32 : 1;
  f32x16 s[HPW];
  half_scores<E, D, HPW, F8>(a, Kl, ks0, qw, q, qf, pat, eo, s);
  // The softmax below is vector work; at a higher priority than the score products of a wave
  // that shares the SIMD, it issues while that wave's products wait for the matrix core (a wave
  // whose next product cannot issue otherwise holds up the other wave's vector instructions).
  // Measured at c2 / c4: 25.5 -> 24.8 us / 182 -> 176 us; no change at c3 and c5.
  __builtin_amdgcn_s_setprio(1);
  // V^T operands of O^T += V^T P^T, shared by the heads: read transposed from the
  // row-major V block, keys in the row order of the P^T C tile.
  u32x4 vf[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int t = 0; t < 2; ++t) vf[db][t] = tr_frag_swz<D>(Vl, 16 * t, 32 * db, D);
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    float m = s[h][0];
#pragma unroll
    for (int e = 1; e < 16; ++e) m = fmaxf(m, s[h][e]);
    const float mx = max_halves(m) * a.c;  // row max in the log2 domain (-inf stays -inf)
    // Lazy rescaling: the exponent reference m2 moves only when some row's maximum
    // exceeds it by more than kRescaleGap, so P <= 2^kRescaleGap and the rescale of the
    // accumulators is skipped on most steps.  Results are the same up to rounding.
    if (wave_any(mx > m2[h] + kRescaleGap)) {
      const float mnew = fmaxf(m2[h], mx);
      const float alpha = mnew == kNegInf ? 1.f : fast_exp2(m2[h] - mnew);
      m2[h] = mnew;
      lsum[h] *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[h][db] *= alpha;
    }
    const float ms = m2[h] == kNegInf ? 0.f : m2[h];
    float sv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) sv[e] = fast_exp2(fmaf(s[h][e], a.c, -ms));
    const u32x4 pb0 = pack8<E>(sv), pb1 = pack8<E>(sv + 8);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      acc[h][db] = E::mfma(vf[db][0], pb0, acc[h][db]);
      acc[h][db] = E::mfma(vf[db][1], pb1, acc[h][db]);
    }
    // the row sum adds the 16-bit P that the PV product uses
#pragma unroll
    for (int w = 0; w < 4; ++w) lsum[h] = E::sum2(pb0[w], lsum[h]);
#pragma unroll
    for (int w = 0; w < 4; ++w) lsum[h] = E::sum2(pb1[w], lsum[h]);
  }
  __builtin_amdgcn_s_setprio(0);
}

// fwd_half for the sliding forward's separate sink half with S <= 8: keys [0, 32), none of them in
// a row's window and every row past key 31, so only keys [0, 8) can be allowed -- registers 0..3
// of each lane (keys 4hf + e).  Their P is computed, the rest is 0, and O^T += V^T P^T takes keys
// [0, 16) only (one product per 32 columns instead of two).
template <typename E, int D, int HPW>
__device__ __forceinline__ void fwd_sink_half8(const Args& a, const uint16_t* Kl, const uint16_t* Vl,
                                               const u32x4 (&qf)[HPW][kQFrags<D, 0>], float (&m2)[HPW],
                                               float (&lsum)[HPW], f32x16 (&acc)[HPW][D >= 32 ? D / 32 : 1]) {
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int KS = kQFrags<D, 0>;
  const int lane = threadIdx.x & 63;
  const int r32 = lane & 31, hf = lane >> 5;
  u32x4 kf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const u32x4*>(Kl + swz_off<D>(r32, hf * (D / 2) + 8 * ks));
  f32x16 s[HPW];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    s[h] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s[h] = E::mfma(kf[ks], qf[h][ks], s[h]);
  }
  u32x4 vf[DB];  // V^T over keys [0, 16)
#pragma unroll
  for (int db = 0; db < DB; ++db) vf[db] = tr_frag_swz<D>(Vl, 0, 32 * db, D);
  bool ok[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) ok[e] = 4 * hf + e < a.S;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    float m = kNegInf;
#pragma unroll
    for (int e = 0; e < 4; ++e) m = ok[e] ? fmaxf(m, s[h][e]) : m;
    const float mx = max_halves(m) * a.c;  // key 0 is allowed on every row: finite
    if (wave_any(mx > m2[h] + kRescaleGap)) {  // (fwd_half's lazy rescaling)
      const float mnew = fmaxf(m2[h], mx);
      const float alpha = mnew == kNegInf ? 1.f : fast_exp2(m2[h] - mnew);
      m2[h] = mnew;
      lsum[h] *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[h][db] *= alpha;
    }
    const float ms = m2[h] == kNegInf ? 0.f : m2[h];
    float sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sv[e] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pe = fast_exp2(fmaf(s[h][e], a.c, -ms));
      sv[e] = ok[e] ? pe : 0.f;
    }
    const u32x4 pb0 = pack8<E>(sv);
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[h][db] = E::mfma(vf[db], pb0, acc[h][db]);
    lsum[h] = E::sum2(pb0[0], lsum[h]);
    lsum[h] = E::sum2(pb0[1], lsum[h]);
  }
}

// P V on the fp8 matrix cores (F8 = 2): one 64-key block [kb, kb + 64) -- swizzled e4m3 K and V
// tiles at Kl, Vl, both laid out like 16-bit rows of D / 2 elements -- for the HPW heads of the
// wave.  v_mfma_scale_f32_32x32x64 reduces over 64 keys, so both halves' scores come first (a half
// with need[sb] false lies outside the wave's rows and counts as masked), then one online-softmax
// update over the 64 keys.
//  * P = 2^(s c - m2 + kP8Shift) is rounded to e4m3.  m2 moves when a row's maximum exceeds it by
//    more than kP8Gap, so P <= 2^(kP8Gap + kP8Shift) = 256 < 448, the e4m3 maximum; weights down
//    to 2^-(kP8Shift + 9) of the row maximum's stay representable.
//  * The row sum adds the rounded P that the product uses, so every row's weights sum to one.  It
//    runs on the matrix cores too: a product with an all-ones A operand leaves the sum of row q's
//    64 weights in every register of column q, accumulated in lacc like O^T in acc.
//  * Packed word w of lane (q, hf) holds P of keys 8w + 4hf + 0..3 (the C layout of S^T); one
//    v_permlane32_swap per word pair turns that into keys 16m + 8hf + 0..7 in words 2m, 2m + 1,
//    runs of 8 keys that ds_read_b64_tr_b8 reads from the row-major V tile as the A operand.
constexpr float kP8Gap = 4.f, kP8Shift = 4.f;

template <int D, int HPW>
__device__ __forceinline__ void fwd_block_pv8(const Args& a, const uint16_t* Kl, const uint16_t* Vl, int kb,
                                              const bool (&need)[2], int qw, int q,
                                              const u32x4 (&qf)[HPW][D / 32], float (&m2)[HPW],
                                              f32x16 (&lacc)[HPW], f32x16 (&acc)[HPW][D / 32], const float* pat,
                                              EdgeOffsets eo) {
  constexpr int DB = D / 32;
  const int lane = threadIdx.x & 63;
  f32x16 s[2][HPW];
#pragma unroll
  for (int sb = 0; sb < 2; ++sb)
    if (need[sb]) half_scores<BF16, D, HPW, 2>(a, Kl + 32 * sb * (D / 2), kb + 32 * sb, qw, q, qf, pat, eo, s[sb]);
  __builtin_amdgcn_s_setprio(1);  // (as fwd_half: the softmax and P V above the score products)
  // V^T operands, shared by the heads: lane (r, hf) byte 8m + t is V[16m + 8hf + t][32db + r].
  // Lane 2j + b of 16-lane group g addresses key 16m + 8(g / 2) + j, bytes 32db + 16(g % 2) + 8b.
  u32x4 vf[DB][2];
  {
    const int g = lane >> 4, sl = lane & 15;
    const int key = 8 * (g >> 1) + (sl >> 1);
    const int col = 8 * (g & 1) + 4 * (sl & 1);  // in 16-bit units
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const u32x2 x = ds_read_tr8(Vl + swz_off<D / 2>(key + 16 * m, 16 * db + col));
        vf[db][m / 2][2 * (m % 2)] = x[0];
        vf[db][m / 2][2 * (m % 2) + 1] = x[1];
      }
  }
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    float m = kNegInf;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
      if (need[sb])
#pragma unroll
        for (int e = 0; e < 16; ++e) m = fmaxf(m, s[sb][h][e]);
    const float mx = max_halves(m) * a.c;
    if (wave_any(mx > m2[h] + kP8Gap)) {
      const float mnew = fmaxf(m2[h], mx);
      const float alpha = mnew == kNegInf ? 1.f : fast_exp2(m2[h] - mnew);
      m2[h] = mnew;
      lacc[h] *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[h][db] *= alpha;
    }
    const float ms = (m2[h] == kNegInf ? 0.f : m2[h]) - kP8Shift;
    uint32_t pw[8];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (need[sb]) {
        float sv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) sv[e] = fast_exp2(fmaf(s[sb][h][e], a.c, -ms));
#pragma unroll
        for (int w = 0; w < 4; ++w) pw[4 * sb + w] = pack4_fp8(sv[4 * w], sv[4 * w + 1], sv[4 * w + 2], sv[4 * w + 3]);
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) pw[4 * sb + w] = 0u;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) swap_halves(pw[2 * j], pw[2 * j + 1]);
    const u32x4 plo = {pw[0], pw[1], pw[2], pw[3]}, phi = {pw[4], pw[5], pw[6], pw[7]};
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[h][db] = mfma_fp8(vf[db][0], vf[db][1], plo, phi, acc[h][db]);
    const u32x4 ones = {0x38383838u, 0x38383838u, 0x38383838u, 0x38383838u};  // e4m3 1.0
    lacc[h] = mfma_fp8(ones, ones, plo, phi, lacc[h]);
  }
  __builtin_amdgcn_s_setprio(0);
}


// F8 (e4m3 q, k, v; fa_fwd_fp8 and fa_fwd_fp8_pv): Q K^T runs on the fp8 MFMA and O (type E =
// BF16) is scaled by a.oscale, the dequantisation factor of V.  With F8 = 1, V is widened to bf16
// (exactly) on its way into LDS and P V is the 16-bit path's; with F8 = 2, V stays e4m3 in LDS and
// P V runs on the fp8 MFMA too (fwd_block_pv8).
template <typename E, int D, int HPW, int F8>
__global__ __launch_bounds__(256) void fwd_kernel(const Args a) {
  constexpr int BN = 64;                   // keys per LDS block
  constexpr int KS = kQFrags<D, F8>;       // 16-byte Q fragments per head and lane
  constexpr int DB = D >= 32 ? D / 32 : 1; // 32-row C tiles of O^T
  constexpr int EB = F8 ? 1 : 2;           // bytes per input element
  constexpr int KBUF = BN * D * EB / 2;    // K block in LDS (16-bit units), swizzled row-major [key][d]
  constexpr int BUF = KBUF + (F8 == 2 ? KBUF : BN * D);  // K, then V (16-bit unless F8 = 2), swizzled [key][d]
  constexpr int CPR = D * EB / 16;         // 16-byte chunks per K (or V) row in memory
  constexpr int CPB = BN * CPR;            // 16-byte chunks per 64-key block of K (or V)
  constexpr int NK = (CPB + 255) / 256;    // chunks per thread
  constexpr bool ALL_ON = CPB >= 256;      // every thread loads a chunk of every tile
  constexpr int NX = 8;                    // XCDs: workgroup i runs on XCD i % 8
  // 16-bit D = 128 reads Q straight into registers: a stash would take LDS that a second
  // resident workgroup per CU needs.
  constexpr bool kStash = F8 || D <= 64;
  constexpr int STASH = kStash ? HPW * KS * 512 : 0;  // per wave: the next tile's Q fragments
  // Small head dims (16-bit D <= 32): a block's compute is short next to the latency of fetching
  // the next block, so every block of a tile (up to NBUF at a time) is fetched at once, by LDS DMA,
  // into NBUF buffers, and the blocks are then computed back to back.  Wider heads double-buffer,
  // one block ahead (through registers, or by DMA: KDMA).
  constexpr bool PRE = !F8 && D <= 32;
  // 16-bit D = 128 and the fp8 P V path (e4m3 K and V kept as they are in LDS): key blocks by DMA
  // into the two buffers, one block ahead, instead of through registers (D = 128: 219 instead of
  // 240 VGPRs, c5 forward 204.6 -> 195.2 us; fa_fwd_fp8_pv c3 536 -> 514 us, c5 164 -> 158 us).
  // At 16-bit D = 64 the same form measured 0.8-2.3% slower at full causal, so it keeps the
  // register path, and so does fp8 Q K^T with 16-bit P V (its V is widened on the way to LDS).
  constexpr bool KDMA = (!F8 && D == 128) || F8 == 2;
  constexpr int NBUF = PRE ? 32768 / (2 * BUF) : 2;  // 32 KiB of K/V blocks
  __shared__ __attribute__((aligned(16))) uint16_t lds[NBUF * BUF + 4 * STASH + 2 * kPatterns * kPatternFloats];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform in a scalar register, so that per-wave rows, heads and buffer descriptors stay
  // scalar (no per-lane copies, no waterfall loops around buffer loads)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int W = a.W, S = a.S;

  // this workgroup's tiles: its XCD's contiguous range [t_lo, t_hi), walked in rounds of wgs_x
  // consecutive tiles, one per workgroup (neighbouring tiles share K/V rows in that XCD's L2).
  // Round r gives workgroup pos the tile pos for even r and wgs_x - 1 - pos for odd r: a causal
  // tile's work grows with its row, and the alternation gives every workgroup about the same sum
  // (with a fixed stride the last workgroup of an XCD got 1.66x the first's at full causal).
  const int hwg = HPW * a.wh;
  const int n_tiles = a.n_qtiles * a.B * (a.Hq / hwg);
  const int xcd = blockIdx.x % NX, pos = blockIdx.x / NX, wgs_x = gridDim.x / NX;
  const int per = n_tiles / NX, rem = n_tiles % NX;
  const int t_lo = xcd * per + min(xcd, rem), t_hi = t_lo + per + (xcd < rem ? 1 : 0);

  // tile -> (b, KV head, this wave's first head hw, first row of the tile q0 and of the wave qw,
  // the sequence's length L and first row)
  struct TileIdx {
    int b, kvh, hw, q0, qw, L;
    int64_t row;
  };
  // Tile order, slowest first: KV head, batch, head group of the KV head, row tile.  The KV head
  // is outermost so that the XCD ranges split over KV heads before they split over sequences:
  // with at least 8 KV heads every XCD gets the same sequences, so the work stays even when the
  // sequences of a variable-length batch differ in length (their tiles past the end are empty).
  auto decode = [&](int tile) {
    KArgs& A = args_fresh();
    TileIdx t;
    const int qt = tile % A.n_qtiles, hg = tile / A.n_qtiles;
    const int gpk = A.G / hwg;  // head groups per KV head
    const int bk = hg / gpk;
    t.b = bk % A.B;
    t.kvh = bk / A.B;
    const Seq sq = seq_of(A, t.b);
    t.L = sq.L;
    t.row = sq.row;
    const int h0 = t.kvh * A.G + (hg % gpk) * hwg;
    t.q0 = qt * 32 * A.wq;
    t.qw = t.q0 + 32 * (wave % A.wq);
    t.hw = h0 + HPW * (wave / A.wq);
    return t;
  };

  // A tile's Q rows for this wave go by LDS DMA into the wave's own stash -- fragment (h, ks)
  // of lane l at 16 bytes each, in lane order -- so they occupy no registers while the current
  // tile computes.  Buffer resources over the sequence's rows [0, L) of the head: rows past L
  // read as zero.
  uint16_t* stash = lds + NBUF * BUF + wave * STASH;
  auto q_rsrc = [&](const TileIdx& t, int h) {
    KArgs& A = args_fresh();
    return make_rsrc(reinterpret_cast<const char*>(A.q) + EB * slice_off(A.sq, t.b, t.hw + h, t.row),
                     span_bytes(t.L, A.sq[2], D, EB));
  };
  auto q_off = [&](const TileIdx& t, int ks) {
    if constexpr (F8)
      return uint32_t(int64_t(t.qw + r32) * args_fresh().sq[2] + 64 * (ks / 2) + 32 * hf + 16 * (ks % 2));
    else
      return uint32_t((int64_t(t.qw + r32) * args_fresh().sq[2] + hf * (D / 2) + 8 * ks) * 2);
  };
  auto stash_rows = [&](const TileIdx& t) {
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const rsrc_t rq = q_rsrc(t, h);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) buf_dma16(rq, stash + (h * KS + ks) * 512, q_off(t, ks));
    }
  };

  // K/V staging offsets of the thread's first chunk (the same for every tile); chunk it lies
  // RSTEP rows further, which keeps the swizzle (it depends on the row mod 8 only).  e4m3 K rows
  // go to LDS as they are (swizzled like 16-bit rows of D / 2 elements); e4m3 V chunks become
  // two 16-bit chunks of the 16-bit V tile.
  constexpr int RSTEP = 256 / CPR;
  const int row0 = tid / CPR, col0 = tid % CPR;
  const uint32_t off_k0 = uint32_t(int64_t(row0) * a.sk[2] * EB + 16 * col0);
  const uint32_t off_v0 = uint32_t(int64_t(row0) * a.sv[2] * EB + 16 * col0);
  const int off_l0 = F8 ? swz_off<D / 2>(row0, 8 * col0) : swz_off<D>(row0, 8 * col0);
  const int off_lv0 = F8 == 1 ? swz_off<D>(row0, 16 * col0) : off_l0;
  const int off_lv1 = F8 == 1 ? swz_off<D>(row0, 16 * col0 + 8) : off_l0;
  const uint32_t bk = uint32_t(EB * a.sk[2]), bv = uint32_t(EB * a.sv[2]);  // bytes per key row

  // the recurring masks (made visible by the barrier before the first key block)
  float* const pat = reinterpret_cast<float*>(lds + NBUF * BUF + 4 * STASH);
  fwd_patterns(pat, W, S);
  const EdgeOffsets eo = edge_offsets(W);

  const int first_tile = t_lo + pos;
  // from a round's tile to the next round's: 2 wgs_x - 1 - 2 pos after an even round, 2 pos + 1
  // after an odd one
  int step = 2 * wgs_x - 1 - 2 * pos;
  // (PRE loads the first tile's Q rows in the loop, in the same round trip as its key blocks)
  if (kStash && !PRE && first_tile < t_hi) {
    stash_rows(decode(first_tile));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  // Only the last round can be short, so the first tile past the range ends the walk.  (A step
  // rather than a round counter: with a counter, the register allocator made the D <= 32 kernels
  // wait for their first argument load before issuing the next, 0.3 us more at c1.)
  for (int tile = first_tile; tile < t_hi; tile += step, step = 2 * wgs_x - step) {
  const int next_tile = tile + step;
  const bool has_next = next_tile < t_hi;
  const TileIdx t = decode(tile);
  const int b = t.b, kvh = t.kvh, hw = t.hw, q0 = t.q0, qw = t.qw, L = t.L;
  const int BM = 32 * a.wq;
  const int q = qw + r32;
  const bool wave_active = qw < L;

  // Q^T operand fragments, from the stash (this wave's own DMA, complete by now: see the wait
  // after the key loop) or from memory: lane (q, hf) holds head-dim slice [hf*D/2 + 8ks, +8) in
  // step ks.
  u32x4 qf[HPW][KS];
  auto read_q = [&]() {
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      if constexpr (kStash) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[h][ks] = lds16(stash + (h * KS + ks) * 512 + 8 * lane) ^ a.qsign;
      } else {
        const rsrc_t rq = q_rsrc(t, h);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[h][ks] = buf_ld16(rq, q_off(t, ks)) ^ a.qsign;
      }
    }
  };
  if (!PRE) read_q();

  float m2[HPW], lsum[HPW];
  f32x16 acc[HPW][DB];
  f32x16 lacc[F8 == 2 ? HPW : 1];  // F8 = 2: row sums from the matrix cores (fwd_block_pv8)
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    m2[h] = kNegInf;
    lsum[h] = 0.f;
    if constexpr (F8 == 2) lacc[h] = f32x16{};
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[h][db] = f32x16{};
  }

  // Key block enumeration for the workgroup's rows [q0, q_end).
  const QPlan plan = qplan(q0, BM, L, W, S);

  // K/V of the KV head through buffer resources spanning the sequence's rows [0, L): rows past L
  // read as zero, so the loads need no branches (a slice is < 2^31 bytes, checked by the C ABI).
  KArgs& Akv = args_fresh();
  const rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(Akv.k) + EB * slice_off(Akv.sk, b, kvh, t.row),
                              span_bytes(L, Akv.sk[2], D, EB));
  const rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(Akv.v) + EB * slice_off(Akv.sv, b, kvh, t.row),
                              span_bytes(L, Akv.sv[2], D, EB));

  // Register staging of the next LDS block.
  u32x4 kreg[NK], vreg[NK];
  auto gload = [&](int kb) {
#pragma unroll
    for (int it = 0; it < NK; ++it) {
      if (ALL_ON || tid + 256 * it < CPB) {
        kreg[it] = buf_ld16(rk, off_k0 + uint32_t(kb + RSTEP * it) * bk);
        vreg[it] = buf_ld16(rv, off_v0 + uint32_t(kb + RSTEP * it) * bv);
      }
    }
  };
  auto sstore = [&](int buf) {
    uint16_t* Kl = lds + buf * BUF;
    uint16_t* Vl = Kl + KBUF;
#pragma unroll
    for (int it = 0; it < NK; ++it) {
      if (ALL_ON || tid + 256 * it < CPB) {
        if constexpr (F8 == 2) {
          st16(Kl + off_l0 + RSTEP * (D / 2) * it, kreg[it]);
          st16(Vl + off_l0 + RSTEP * (D / 2) * it, vreg[it]);
        } else if constexpr (F8) {
          st16(Kl + off_l0 + RSTEP * (D / 2) * it, kreg[it]);
          u32x4 v0, v1;
          fp8x16_to_bf16(vreg[it], v0, v1);
          st16(Vl + off_lv0 + RSTEP * D * it, v0);
          st16(Vl + off_lv1 + RSTEP * D * it, v1);
        } else {
          st16(Kl + off_l0 + RSTEP * D * it, kreg[it]);
          st16(Vl + off_l0 + RSTEP * D * it, vreg[it]);
        }
      }
    }
  };

  // one key block [kb, kb + 64) from LDS buffer `buf`
  auto compute_block = [&](int kb, int buf) {
    if (!wave_active) return;
    const uint16_t* Kl = lds + buf * BUF;
    const uint16_t* Vl = Kl + KBUF;
    if constexpr (F8 == 2) {
      const bool need[2] = {wave_needs(kb, qw, L, W, S), wave_needs(kb + 32, qw, L, W, S)};
      if (need[0] || need[1]) fwd_block_pv8<D, HPW>(a, Kl, Vl, kb, need, qw, q, qf, m2, lacc, acc, pat, eo);
    } else {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int ks0 = kb + 32 * sb;
        if (!wave_needs(ks0, qw, L, W, S)) continue;
        fwd_half<E, D, HPW, F8>(a, Kl + 32 * sb * (KBUF / BN), Vl + 32 * sb * D, ks0, qw, q, qf, m2, lsum, acc,
                                pat, eo);
      }
    }
  };

  // DMA of a 64-key block into buffer j: the block's K and V tiles are CPB 16-byte chunks each,
  // 2 CPB / 64 instructions of 64 lanes; wave w issues instructions [w NIW, (w + 1) NIW), and lane
  // l of instruction p (of K or V) loads the chunk that the swizzle places at position 64 p + l
  constexpr int IPT = CPB / 64;       // instructions per tile (K or V)
  constexpr int NIW = 2 * IPT / 4;    // per wave
  static_assert(!(PRE || KDMA) || (NIW >= 1 && 2 * IPT == 4 * NIW), "whole instructions per wave");
  auto dma_block = [&](int kb, int j) {
#pragma unroll
    for (int n = 0; n < NIW; ++n) {
      const int ii = wave * NIW + n, is_v = ii >= IPT, pi = is_v ? ii - IPT : ii;
      const int pos = 64 * pi + lane, row = pos / CPR, col = (pos % CPR) ^ swz<F8 ? D / 2 : D>(row);
      uint16_t* dst = lds + j * BUF + (is_v ? KBUF : 0) + 512 * pi;
      const uint32_t off = uint32_t(int64_t(kb + row) * (is_v ? bv : bk)) + 16u * uint32_t(col);
      if (is_v) buf_dma16(rv, dst, off);
      else buf_dma16(rk, dst, off);
    }
  };
  if constexpr (PRE) {
    if (plan.nb == 0) {  // no key block: the Q rows are still read out of the stash
      if (kStash && tile == first_tile) {
        stash_rows(t);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      read_q();
    }
    for (int g0 = 0; g0 < plan.nb; g0 += NBUF) {
      const int ng = min(NBUF, plan.nb - g0);
      for (int j = 0; j < ng; ++j) dma_block(qplan_block(plan, g0 + j), j);
      if (g0 == 0) {
        if (kStash && tile == first_tile) {  // the first tile's Q rows, with its first blocks
          stash_rows(t);
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        read_q();
      }
      // the next tile's Q rows into the stash, once this tile's have been read out of it
      const bool stash_now = kStash && g0 == 0 && has_next;
      if (stash_now) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        stash_rows(decode(next_tile));
        wait_vm_lgkm0_barrier<HPW * KS>();  // the blocks have landed (the stash may be in flight)
      } else {
        wait_vm_lgkm0_barrier<0>();
      }
      for (int j = 0; j < ng; ++j) compute_block(qplan_block(plan, g0 + j), j);
      __syncthreads();  // before the buffers are refilled
    }
  } else if constexpr (KDMA) {
    // block i in buffer i & 1; block i + 1's DMA is issued before block i computes (its buffer was
    // last read by block i - 1, behind the barrier that ended it) and waited for after it; the next
    // tile's Q rows (HPW KS loads, issued after it in block 0) may stay in flight past that wait
    if (plan.nb > 0) {
      dma_block(qplan_block(plan, 0), 0);
      wait_vm_lgkm0_barrier<0>();
    }
    for (int i = 0; i < plan.nb; ++i) {
      const bool more = i + 1 < plan.nb;
      if (more) dma_block(qplan_block(plan, i + 1), (i + 1) & 1);
      const bool stash_now = kStash && i == 0 && has_next;
      if (stash_now) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        stash_rows(decode(next_tile));
      }
      compute_block(qplan_block(plan, i), i & 1);
      if (stash_now) wait_vm_lgkm0_barrier<HPW * KS>();
      else wait_vm_lgkm0_barrier<0>();
    }
  } else {
    if (plan.nb > 0) {  // (a tile past its sequence's end, in a variable-length batch, has none)
      gload(qplan_block(plan, 0));
      sstore(0);
      __syncthreads();
    }
    for (int i = 0; i < plan.nb; ++i) {
      const bool more = i + 1 < plan.nb;
      if (more) gload(qplan_block(plan, i + 1));
      // the next tile's Q rows into the stash, once this tile's have been read out of it
      if (kStash && i == 0 && has_next) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        stash_rows(decode(next_tile));
      }
      compute_block(qplan_block(plan, i), i & 1);
      if (more) sstore((i + 1) & 1);
      __syncthreads();
    }
  }
  if (kStash && plan.nb == 0 && has_next) {  // no key block: stash it here
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    stash_rows(decode(next_tile));
  }
  // the next tile's stash has landed (waited here, before this tile's O stores, which would
  // otherwise also be waited for)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if (!wave_active) continue;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    float lt;
    if constexpr (F8 == 2)  // the whole row's sum, of P scaled by 2^kP8Shift
      lt = lacc[h][0] * (1.f / (1 << int(kP8Shift)));
    else
      lt = sum_halves(lsum[h]);
    if (q >= L) continue;
    float mt = m2[h], r = 1.f;
    KArgs& A = args_fresh();
    if (A.sink_logits) {
      // the learned sink joins the denominator: l' = l 2^(m - m') + 2^(sink*log2e - m'), with
      // m' = max(m, sink*log2e) so that neither term overflows
      const float sl = A.sink_logits[hw + h] * kLog2e;
      const float mn = fmaxf(mt, sl);
      r = fast_exp2(mt - mn);
      lt = lt * r + fast_exp2(sl - mn);
      mt = mn;
    }
    float inv = lt > 0.f ? r / lt : 0.f;
    if constexpr (F8 == 2) inv *= A.oscale / (1 << int(kP8Shift));
    else if constexpr (F8) inv *= A.oscale;
    char* op = reinterpret_cast<char*>(A.o_out) + 2 * slice_off(A.so_out, b, hw + h, t.row + q);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      if (D == 16 && hf == 1) continue;
      float ov[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) ov[e] = acc[h][db][e] * inv;
      if constexpr (F8 == 2) {  // C row 8j + 4hf + i is head dim 32db + 8j + 4hf + i
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x2 w = {E::pack2(ov[4 * j], ov[4 * j + 1]), E::pack2(ov[4 * j + 2], ov[4 * j + 3])};
          *reinterpret_cast<u32x2*>(op + 2 * (32 * db + 8 * j + 4 * hf)) = w;
        }
        continue;
      }
      const int d0 = 32 * db + (D >= 32 ? 16 * hf : 0);
      st16(op + 2 * d0, pack8<E>(ov));
      st16(op + 2 * (d0 + 8), pack8<E>(ov + 8));
    }
    if (hf == 0) {
      A.lse_out[slice_off(A.slse, b, hw + h, t.row + q)] =
          (mt + fast_log2(lt)) * kLn2;
    }
  }
  }  // tiles
}

// ---------------------------------------------------------------------------------------------
// Sliding forward, for the GPT-OSS sliding layers (16-bit, D = 64, KV groups of a multiple of 8
// query heads, 1 <= W <= 129, S <= 32; the C ABI's plan_fwd_slide checks): the forward twin of
// bwd_dq_slide_kernel (fa_bwd_slide.hip).  A workgroup is 4 waves x 2 heads -- the 8 query heads
// of one head group -- and walks slide_ct consecutive 32-row tiles.  Tile m visits the sink half
// (when slide_sink_half) and the window halves slide_hlo(m, W) .. m, all resident in an LDS ring
// of kFwdSlideRing slots (half j in slot j % kFwdSlideRing) plus a sink slot; tile m brings in one
// half, the next tile's diagonal half m + 1, by LDS DMA into the slot that its own halves
// m - 4 .. m leave free.  The next tile's Q rows are loaded into registers while the current tile
// computes.  LDS: 7 slots of K and V (8 KB each) and the mask patterns = 72 KB, two workgroups per
// CU.  The per-half work is fwd_half, the same as fwd_kernel's.
// ---------------------------------------------------------------------------------------------
// VL: a packed batch's enumeration of the units (a separate instantiation, so that the
// fixed-length kernel's code and registers are not touched by it).
template <typename E, bool VL>
__global__ __launch_bounds__(256, 2) void fwd_slide_kernel(const Args a) {
  constexpr int D = 64, HPW = 2, KS = D / 16, DB = D / 32;
  constexpr int TILE = 32 * D;    // one swizzled [32][D] tile of 16-bit values
  constexpr int HALF = 2 * TILE;  // a ring slot: K, then V, of 32 keys
  constexpr int NR = kFwdSlideRing;
  constexpr int CPR = D / 8;
  __shared__ __attribute__((aligned(16))) uint16_t lds[(NR + 1) * HALF + 2 * kPatterns * kPatternFloats];
  uint16_t* const ring = lds;
  float* const pat = reinterpret_cast<float*>(lds + (NR + 1) * HALF);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int W = a.W, S = a.S;

  // unit -> (KV head, batch, head group, chunk), chunks fastest (as bwd_dq_slide_kernel); a packed
  // batch hands out only the chunks with rows: (KV head, head group), then each sequence's chunks
  const int hg_n = a.G / 8;
  const int unit = xcd_remap(blockIdx.x, gridDim.x);
  int chunk, hg, b, kvh;
  if constexpr (VL) {
    const int grp = unit / a.vl_units;
    hg = grp % hg_n;
    kvh = grp / hg_n;
    if (!varlen_nth(a, unit % a.vl_units, a.vl_units, 32, a.slide_ct, b, chunk)) return;
  } else {
    chunk = unit % a.slide_ncu;
    const int rest = unit / a.slide_ncu;
    hg = rest % hg_n;
    const int bk = rest / hg_n;
    b = bk % a.B;
    kvh = bk / a.B;
  }
  const Seq sq = seq_of(a, b);
  const int L = sq.L;
  const int n_qt = (L + 31) / 32;
  const int qt0 = chunk * a.slide_ct;
  const int qt1 = min(qt0 + a.slide_ct, n_qt);
  if (qt0 >= qt1) return;  // past the end of a short sequence (variable-length batches)
  const int hw = kvh * a.G + hg * 8 + HPW * wave;  // this wave's first query head

  // the recurring masks (visible after the first barrier)
  fwd_patterns(pat, W, S);
  const EdgeOffsets eo = edge_offsets(W);

  // Q of the wave's two heads, straight into registers
  rsrc_t rq[HPW];
#pragma unroll
  for (int h = 0; h < HPW; ++h)
    rq[h] = make_rsrc(reinterpret_cast<const char*>(a.q) + 2 * slice_off(a.sq, b, hw + h, sq.row), span_bytes(L, a.sq[2], D));
  const uint32_t sq2 = uint32_t(a.sq[2]);
  u32x4 qn[HPW][KS];
  auto load_q = [&](int qt) {
#pragma unroll
    for (int h = 0; h < HPW; ++h)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qn[h][ks] = buf_ld16(rq[h], (uint32_t(32 * qt + r32) * sq2 + uint32_t(hf * (D / 2) + 8 * ks)) * 2u);
  };

  // K/V halves by DMA: the 8 instructions of a half (K positions 64p + lane for p = 0..3, then V)
  // go two per wave
  const rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(a.k) + 2 * slice_off(a.sk, b, kvh, sq.row), span_bytes(L, a.sk[2], D));
  const rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(a.v) + 2 * slice_off(a.sv, b, kvh, sq.row), span_bytes(L, a.sv[2], D));
  const int64_t skr = a.sk[2], svr = a.sv[2];
  uint32_t kv_off[2];
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const int ii = 2 * wave + n, p = ii & 3;
    const int pos = 64 * p + lane, row = pos / CPR, col = (pos % CPR) ^ swz<D>(row);
    kv_off[n] = uint32_t((int64_t(row) * (ii >= 4 ? svr : skr) + 8 * col) * 2);
  }
  const uint32_t hb_k = uint32_t(32 * skr * 2), hb_v = uint32_t(32 * svr * 2);
  // (asm_dma = std::true_type: issued from inline assembly, which the compiler's waits for the Q
  // loads do not wait for)
  auto load_half = [&](int j, int slot, auto asm_dma) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int ii = 2 * wave + n;
      uint16_t* dst = ring + slot * HALF + (ii >= 4 ? TILE : 0) + 512 * (ii & 3);
      if constexpr (decltype(asm_dma)::value) {
        if (ii >= 4) buf_dma16_asm(rv, dst, kv_off[n] + uint32_t(j) * hb_v);
        else buf_dma16_asm(rk, dst, kv_off[n] + uint32_t(j) * hb_k);
      } else {
        if (ii >= 4) buf_dma16(rv, dst, kv_off[n] + uint32_t(j) * hb_v);
        else buf_dma16(rk, dst, kv_off[n] + uint32_t(j) * hb_k);
      }
    }
  };

  // prologue: the first tile's Q, the sink half and the first tile's window halves
  load_q(qt0);
  if (S > 0) load_half(0, NR, std::false_type{});
  for (int j = slide_hlo(qt0, W); j <= qt0; ++j) load_half(j, j % NR, std::false_type{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  for (int qt = qt0; qt < qt1; ++qt) {
    const int qw = 32 * qt, q = qw + r32;
    const bool has_next = qt + 1 < qt1;
    // every wave's share of this tile's halves has landed (each waited for its own loads before
    // its O stores); in the first tile, the patterns are written
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // this tile's Q rows, before the next tile's loads: the compiler's wait for the Q loads (already
    // complete) must not also wait for the next half's DMA, which is therefore issued from inline
    // assembly after the copy (the empty statements keep the copy ahead of it)
    u32x4 qf[HPW][KS];
#pragma unroll
    for (int h = 0; h < HPW; ++h)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qf[h][ks] = qn[h][ks] ^ a.qsign;
        asm volatile("" : "+v"(qf[h][ks]));
      }
    if (has_next) {
      load_half(qt + 1, (qt + 1) % NR, std::true_type{});
      load_q(qt + 1);
    }

    float m2[HPW], lsum[HPW];
    f32x16 acc[HPW][DB];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      m2[h] = kNegInf;
      lsum[h] = 0.f;
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[h][db] = f32x16{};
    }
    if (slide_sink_half(qt, W, S)) {
      if (S <= 8) fwd_sink_half8<E, D, HPW>(a, ring + NR * HALF, ring + NR * HALF + TILE, qf, m2, lsum, acc);
      else fwd_half<E, D, HPW, 0>(a, ring + NR * HALF, ring + NR * HALF + TILE, 0, qw, q, qf, m2, lsum, acc, pat, eo);
    }
    for (int j = slide_hlo(qt, W); j <= qt; ++j) {
      if (!wave_needs(32 * j, qw, L, W, S)) continue;
      const uint16_t* Kl = ring + (j % NR) * HALF;
      fwd_half<E, D, HPW, 0>(a, Kl, Kl + TILE, 32 * j, qw, q, qf, m2, lsum, acc, pat, eo);
    }
    // the next tile's half and Q have landed (waited before the O stores, which the next tile
    // does not wait for)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      float lt = sum_halves(lsum[h]);
      if (q >= L) continue;
      float mt = m2[h], r = 1.f;
      KArgs& A = args_fresh();
      if (A.sink_logits) {
        const float sl = A.sink_logits[hw + h] * kLog2e;
        const float mn = fmaxf(mt, sl);
        r = fast_exp2(mt - mn);
        lt = lt * r + fast_exp2(sl - mn);
        mt = mn;
      }
      const float inv = lt > 0.f ? r / lt : 0.f;
      char* op = reinterpret_cast<char*>(A.o_out) + 2 * slice_off(A.so_out, b, hw + h, sq.row + q);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        float ov[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) ov[e] = acc[h][db][e] * inv;
        const int d0 = 32 * db + 16 * hf;
        st16(op + 2 * d0, pack8<E>(ov));
        st16(op + 2 * (d0 + 8), pack8<E>(ov + 8));
      }
      if (hf == 0) A.lse_out[slice_off(A.slse, b, hw + h, sq.row + q)] = (mt + fast_log2(lt)) * kLn2;
    }
  }
}

template <typename E>
static hipError_t launch_fwd_slide_e(const Args& a, hipStream_t stream) {
  const int per = a.vl_units ? a.vl_units : a.B * a.slide_ncu;  // units per (KV head, head group)
  const dim3 grid(unsigned(a.Hkv * (a.G / 8) * per)), block(256);
  if (a.vl_units) hipLaunchKernelGGL((fwd_slide_kernel<E, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((fwd_slide_kernel<E, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_fwd_slide(const Args& a, int dtype, hipStream_t stream) {
  return dtype == 1 ? launch_fwd_slide_e<BF16>(a, stream) : launch_fwd_slide_e<F16>(a, stream);
}

// Resident workgroups per CU of a kernel, remembered per kernel (it depends only on the
// kernel's resources).
template <auto Kernel>
static int fwd_resident_per_cu() {
  static int cached = 0;  // benign race: every thread computes the same value
  if (cached == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, Kernel, 256, 0) != hipSuccess || n < 1) n = 1;
    cached = n;
  }
  return cached;
}

template <typename E, int D, int HPW, int F8 = 0>
static hipError_t launch_fwd_h(const Args& a, hipStream_t stream) {
  const int n_tiles = a.n_qtiles * (a.B * a.Hq / (HPW * a.wh));
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < 1)
    cus = 256;
  // one resident wave of workgroups, a multiple of the 8 XCDs
  const int slots = fwd_resident_per_cu<fwd_kernel<E, D, HPW, F8>>() * cus;
  const int wgs = 8 * ((min(n_tiles, slots) + 7) / 8);
  hipLaunchKernelGGL((fwd_kernel<E, D, HPW, F8>), dim3(wgs), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <typename E, int D>
static hipError_t launch_fwd_d(const Args& a, int hpw, hipStream_t stream) {
  return hpw == 2 ? launch_fwd_h<E, D, 2>(a, stream) : launch_fwd_h<E, D, 1>(a, stream);
}

template <typename E>
static hipError_t launch_fwd_e(const Args& a, int D, int hpw, hipStream_t stream) {
  switch (D) {
    case 16: return launch_fwd_d<E, 16>(a, hpw, stream);
    case 32: return launch_fwd_d<E, 32>(a, hpw, stream);
    case 64: return launch_fwd_d<E, 64>(a, hpw, stream);
    case 128: return launch_fwd_d<E, 128>(a, hpw, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_fwd(const Args& a, int dtype, int D, int hpw, hipStream_t stream) {
  return dtype == 1 ? launch_fwd_e<BF16>(a, D, hpw, stream) : launch_fwd_e<F16>(a, D, hpw, stream);
}

// e4m3 inputs, bf16 output: D = 64 shares K/V fragments between two heads per wave where the
// group size allows, D = 128 has one head per wave.  fp8_pv selects P V on the fp8 MFMA.
template <int F8>
static hipError_t launch_fwd_fp8_m(const Args& a, int D, int hpw, hipStream_t stream) {
  if (D == 64) return hpw == 2 ? launch_fwd_h<BF16, 64, 2, F8>(a, stream) : launch_fwd_h<BF16, 64, 1, F8>(a, stream);
  if (D == 128 && hpw == 1) return launch_fwd_h<BF16, 128, 1, F8>(a, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_fwd_fp8(const Args& a, int D, int hpw, bool fp8_pv, hipStream_t stream) {
  return fp8_pv ? launch_fwd_fp8_m<2>(a, D, hpw, stream) : launch_fwd_fp8_m<1>(a, D, hpw, stream);
}

}  // namespace fa
