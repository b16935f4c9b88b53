// fa_bwd_slide.hip - dQ of the sliding-window backward with K/V resident in an LDS ring.
//
// Same mathematics and outputs as bwd_dq_kernel (fa_bwd.hip; the reference's _backward_dq_kernel,
// benchmark_backward_speed.py:312-387): delta = rowsum(dO o O) and the row statistics for the dK/dV
// kernel, dQ = scale * sum_k P (dP - delta) K over the sink and window keys, and in dq_sink_mode the
// sink keys' dK/dV contributions of the rows past key block 0's window.  It runs instead of
// bwd_dq_kernel for the GPT-OSS sliding layers: D = 64, 16-bit inputs, a group of 8 query heads per
// KV head (G a multiple of 8), 1 <= W <= 161, S <= 32 (the C ABI's plan_slide checks).
//
// A workgroup is 8 waves -- the 8 query heads of one head group of a KV head -- and walks
// slide_ct consecutive 32-row tiles of its sequence.  Tile m (rows [32m, 32m + 32)) needs the
// window keys [32m - W + 1, 32m + 31], i.e. the 32-key halves hlo(m) .. m with
// hlo(m) = max(0, m - ceil((W - 1) / 32)) (at most 6 halves for W <= 161), plus the sink half
// (keys [0, 32)) when that is not among them.  The halves live in an LDS ring of 7 slots (half j
// in slot j % 7) and a sink slot; each tile brings in one new half -- the next tile's diagonal half
// m + 1, by LDS DMA issued at the start of tile m into slot (m + 1) % 7, which tile m does not use
// (its halves occupy the 6 slots of m - 5 .. m) -- so the 8 heads share one copy of K/V and a
// tile stages 8 KB of K/V instead of re-staging its whole window.  The rows of the next tile
// (Q, dO, O) go into each wave's stash by DMA as in bwd_dq_kernel.
//
// LDS: 8 stashes (Q, dO, O of 32 rows, 12 KB each) + 8 slots (K and V of 32 keys, 8 KB each)
// = 160 KB: one workgroup (8 waves, two per SIMD) per CU.
#include "fa_args.h"
#include "fa_common.h"

namespace fa {

namespace {

constexpr int kSlideWaves = 8;
constexpr int kRing = kSlideRing;  // window slots (fa_plan.h); slot kRing holds the sink half

}  // namespace

// VL: a packed batch's enumeration of the units (a separate instantiation, so that the
// fixed-length kernel's code and registers are not touched by it).
template <typename E, bool SINK, bool VL>
__global__ __launch_bounds__(512, 1) void bwd_dq_slide_kernel(const Args a) {
  constexpr int D = 64;
  constexpr int KS = D / 16;
  constexpr int DB = D / 32;
  constexpr int TILE = 32 * D;      // one swizzled [32][D] tile of 16-bit values
  constexpr int STASH = 3 * TILE;   // per wave: Q, dO, O of the next tile
  constexpr int HALF = 2 * TILE;    // per slot: K, then V, of 32 keys
  constexpr int NB16 = D / 16;
  constexpr int CPR = D / 8;        // 16-byte chunks per row
  __shared__ __attribute__((aligned(16))) uint16_t lds[kSlideWaves * STASH + (kRing + 1) * HALF];
  uint16_t* const ring = lds + kSlideWaves * STASH;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int W = a.W, S = a.S;

  // unit -> (KV head, batch, head group, chunk), chunks fastest; a contiguous range of units per
  // XCD, so the chunks of one (batch, KV head) share that XCD's L2.  A packed batch hands out only
  // the chunks with rows: (KV head, head group), then each sequence's chunks.  `slot` is the unit's
  // index in the (KV head, batch, head group, chunk) enumeration either way: its sink-key partials
  // go to slot `slot`, where the folds look for them.
  const int hg_n = a.G / kSlideWaves;
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
  const int slot = VL ? ((kvh * a.B + b) * hg_n + hg) * a.slide_ncu + chunk : unit;
  const Seq sq = seq_of(a, b);
  const int L = sq.L;
  const int n_qt = (L + 31) / 32;
  const int qt0 = chunk * a.slide_ct;
  const int qt1 = min(qt0 + a.slide_ct, n_qt);
  if (qt0 >= qt1) return;  // past the end of a short sequence (variable-length batches)
  const int h = kvh * a.G + hg * kSlideWaves + wave;  // this wave's query head
  const float sink_logit = a.sink_logits ? a.sink_logits[h] : 0.f;  // (a scalar load, before any store)

  // ---- the wave's stash: rows of one tile of head h by DMA, as bwd_dq_kernel's stash_rows
  uint16_t* const stash = lds + wave * STASH;
  const rsrc_t rq = make_rsrc(reinterpret_cast<const char*>(a.q) + 2 * slice_off(a.sq, b, h, sq.row), span_bytes(L, a.sq[2], D));
  const rsrc_t rd = make_rsrc(reinterpret_cast<const char*>(a.dout) + 2 * slice_off(a.sdo, b, h, sq.row), span_bytes(L, a.sdo[2], D));
  const rsrc_t ro = make_rsrc(reinterpret_cast<const char*>(a.o) + 2 * slice_off(a.so, b, h, sq.row), span_bytes(L, a.so[2], D));
  const rsrc_t rl = make_rsrc(a.lse + slice_off(a.slse, b, h, sq.row), span_f32(L, a.slse[2]));
  const uint32_t sq2 = uint32_t(a.sq[2]), sdo2 = uint32_t(a.sdo[2]), so2 = uint32_t(a.so[2]);
  uint32_t st_off[KS];  // element offset (row within the tile, column) of this lane's DMA chunks
#pragma unroll
  for (int p = 0; p < KS; ++p) {
    const int tr = (64 * p + lane) / CPR;
    const int col = 8 * (((64 * p + lane) % CPR) ^ swz<D>(tr));
    st_off[p] = uint32_t(tr) << 16 | uint32_t(col);
  }
  // one of the tile's three row tiles (part 0: Q, 1: dO, 2: O), KS instructions
  auto stash_part = [&](int qt, int part) {
    const rsrc_t r = part == 0 ? rq : part == 1 ? rd : ro;
    const uint32_t rs = part == 0 ? sq2 : part == 1 ? sdo2 : so2;
#pragma unroll
    for (int p = 0; p < KS; ++p) {
      uint32_t so = st_off[p];
      asm volatile("" : "+v"(so));  // computed here: hoisted, the offsets of every part stay live
      const uint32_t row = uint32_t(32 * qt) + (so >> 16), col = so & 0xffffu;
      buf_dma16_asm(r, stash + part * TILE + 512 * p, (row * rs + col) * 2);
    }
  };
  auto stash_rows = [&](int qt) {
#pragma unroll
    for (int part = 0; part < 3; ++part) stash_part(qt, part);
  };
  auto load_lse = [&](int qt) { return buf_ldf(rl, uint32_t(32 * qt + r32) * uint32_t(a.slse[2]) * 4u); };

  // ---- K/V halves by DMA: wave w loads 1 KiB of the half (w < 4: K, positions 64w .. 64w + 63 of
  // the swizzled tile; w >= 4: V), so the 8 waves together stage one half per call
  const bool kind_v = wave >= 4;
  const int64_t kv_rs = kind_v ? a.sv[2] : a.sk[2];
  const rsrc_t rkv = kind_v ? make_rsrc(reinterpret_cast<const char*>(a.v) + 2 * slice_off(a.sv, b, kvh, sq.row), span_bytes(L, a.sv[2], D))
                            : make_rsrc(reinterpret_cast<const char*>(a.k) + 2 * slice_off(a.sk, b, kvh, sq.row), span_bytes(L, a.sk[2], D));
  uint32_t kv_off;  // byte offset of this lane's chunk within a 32-key half
  {
    const int pos = 64 * (wave & 3) + lane;
    const int row = pos / CPR, col = (pos % CPR) ^ swz<D>(row);
    kv_off = uint32_t((int64_t(row) * kv_rs + 8 * col) * 2);
  }
  const uint32_t half_bytes = uint32_t(32 * kv_rs * 2);
  // (Every DMA of this kernel is issued from inline assembly: the compiler would wait for DMAs of
  // its own before each transposed LDS read, and wherever it waits for the LSE load; the explicit
  // waits of the tile loop cover them.)
  auto load_half = [&](int j, int slot) {
    buf_dma16_asm(rkv, ring + slot * HALF + (kind_v ? TILE : 0) + 512 * (wave & 3), kv_off + uint32_t(j) * half_bytes);
  };

  // sink accumulators (dq_sink_mode): lane l holds key 4(l/16) + i, head-dim column 16 nb + l % 16
  f32x4 dks[SINK ? NB16 : 1], dvs[SINK ? NB16 : 1];
  if constexpr (SINK) {
#pragma unroll
    for (int nb = 0; nb < NB16; ++nb) {
      dks[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
      dvs[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  const int sink_row0 = dq_sink_row0(L, W);
  uint16_t* const ptile = stash + 2 * TILE;  // P / dS of the sink keys, in the O tile (read for delta only)

  // ---- prologue: the first tile's rows and the sink half (used first), then its window halves,
  // which may still be in flight while the first tile reads its rows and computes the sink half
  stash_rows(qt0);
  float lse_next = load_lse(qt0);
  if (S > 0) load_half(0, kRing);
  const int hlo0 = slide_hlo(qt0, W);
  for (int j = hlo0; j <= qt0; ++j) load_half(j, j % kRing);
  switch (qt0 - hlo0 + 1) {  // window halves issued last: wait for everything before them
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
  }

  for (int qt = qt0; qt < qt1; ++qt) {
    const int qw = 32 * qt, q = qw + r32;
    const bool has_next = qt + 1 < qt1;
    // every wave's loads for this tile have landed (each waited for its own before its stores;
    // in the first tile, all but the window halves)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // this tile's LSE (the compiler waits for its load here, which also waits for every load and
    // store issued before it), then the next tile's diagonal half into the slot this tile does not
    // use, and the next tile's LSE (a spare load of the last tile's in the last tile)
    const float lse2 = q < L ? lse_next * kLog2e : __builtin_inff();
    asm volatile("" ::"v"(lse2));  // (keeps that wait ahead of the DMA)
    if (has_next) load_half(qt + 1, (qt + 1) % kRing);
    lse_next = load_lse(min(qt + 1, qt1 - 1));

    // row operands and statistics from the stash
    const uint16_t* Qs = stash;
    const uint16_t* Ds = stash + TILE;
    const uint16_t* Os = stash + 2 * TILE;
    u32x4 qf[KS], dof[KS];
    float dsum = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int off = swz_off<D>(r32, hf * (D / 2) + 8 * ks);
      qf[ks] = lds16(Qs + off) ^ a.qsign;
      dof[ks] = lds16(Ds + off);
      dsum = dot8<E>(dof[ks], lds16(Os + off), dsum);
    }
    const float delta = sum_halves(dsum);
    const float ndelta = -delta;

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
    // The next tile's rows, once this tile's have been read out of the stash (after the sink half
    // on the sink path, which also reads the stash), in three parts issued between the window
    // halves: issued at once, a wave's 3 KS DMA instructions stall it while the CU's load path
    // takes the whole workgroup's 96 KB.
    int refilled = 0;  // parts issued
    auto refill_part = [&]() {
      if (has_next) {
        switch (refilled) {  // (constant parts: a run-time part index would put the descriptors on the stack)
          case 0:
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            stash_part(qt + 1, 0);
            break;
          case 1: stash_part(qt + 1, 1); break;
          case 2: stash_part(qt + 1, 2); break;
          default: break;
        }
      }
      ++refilled;
    };

    // One 32-key half from LDS: S^T = K Q^T and dP^T - delta = V dO^T - delta (lane = query row),
    // P and dS elementwise, dQ^T += K^T dS^T (bwd_dq_kernel's step).  Returns P and dS of the
    // half's first 16 keys (registers 0..7) for the sink path.
    auto half_step = [&](const uint16_t* Kl, int ks0, float (&p)[16], float (&ds)[16]) {
      const uint16_t* Vl = Kl + TILE;
      u32x4 kf[KS], vf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = swz_off<D>(r32, hf * (D / 2) + 8 * ks);
        kf[ks] = *reinterpret_cast<const u32x4*>(Kl + off);
        vf[ks] = *reinterpret_cast<const u32x4*>(Vl + off);
      }
      f32x16 s, dp;
      auto qk = [&](const f32x16& c0) {
        f32x16 d0;
#pragma unroll
        for (int e = 0; e < 16; ++e) d0[e] = ndelta;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          s = E::mfma(kf[ks], qf[ks], ks == 0 ? c0 : s);
          dp = E::mfma(vf[ks], dof[ks], ks == 0 ? d0 : dp);
        }
      };
      if (tile_full(ks0, qw, W, S)) {
        qk(f32x16{});
      } else {
        f32x16 bias;
        const int dq0 = q - ks0 - 4 * hf;
        if (ks0 >= S || ks0 + 32 <= S) {
          const unsigned lim = ks0 >= S ? unsigned(W) : 0x80000000u;
#pragma unroll
          for (int e = 0; e < 16; ++e) bias[e] = unsigned(dq0 - (8 * (e / 4) + (e % 4))) < lim ? 0.f : kNegInf;
        } else {
          const int sl = S - ks0 - 4 * hf;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int off = 8 * (e / 4) + (e % 4);
            bias[e] = unsigned(dq0 - off) < (off < sl ? 0x80000000u : unsigned(W)) ? 0.f : kNegInf;
          }
        }
        qk(bias);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = fast_exp2(fmaf(s[e], a.c, -lse2));
        ds[e] = p[e] * dp[e];
      }
      const u32x4 d0 = pack8<E>(ds), d1 = pack8<E>(ds + 8);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        acc[db] = E::mfma(tr_frag_swz<D>(Kl, 0, 32 * db, D), d0, acc[db]);
        acc[db] = E::mfma(tr_frag_swz<D>(Kl, 16, 32 * db, D), d1, acc[db]);
      }
    };

    // The sink half with S <= 8 (when it is not a window half: every row's window starts at key
    // 32 or later, and every row is past key 31): only keys [0, 8) can be allowed, which are
    // registers 0..3 of each lane (keys 4hf + e), so P and dS are computed for those four, the
    // rest are 0, and dQ^T += K^T dS^T takes keys [0, 16) only.
    auto sink_half8 = [&](const uint16_t* Kl, float (&p)[16], float (&ds)[16]) {
      const uint16_t* Vl = Kl + TILE;
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = swz_off<D>(r32, hf * (D / 2) + 8 * ks);
        s = E::mfma(*reinterpret_cast<const u32x4*>(Kl + off), qf[ks], s);
        dp = E::mfma(*reinterpret_cast<const u32x4*>(Vl + off), dof[ks], dp);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = 0.f;
        ds[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pe = fast_exp2(fmaf(s[e], a.c, -lse2));
        p[e] = 4 * hf + e < S ? pe : 0.f;
        ds[e] = p[e] * (dp[e] + ndelta);
      }
      const u32x4 d0 = pack8<E>(ds);
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] = E::mfma(tr_frag_swz<D>(Kl, 0, 32 * db, D), d0, acc[db]);
    };

    const int hlo = slide_hlo(qt, W);
    // the sink half, when it is not one of the window halves (its keys >= S are then all masked)
    if (slide_sink_half(qt, W, S)) {
      float p[16], ds[16];
      if (S <= 8) sink_half8(ring + kRing * HALF, p, ds);
      else half_step(ring + kRing * HALF, 0, p, ds);
      if constexpr (SINK) {
        if (qw + 31 >= sink_row0) {
          // P and dS of keys [0, 16) of rows >= sink_row0 into the [32 rows][16 keys] tiles, then
          // dV_s += P^T dO and dK_s += dS^T Q (bwd_dq_kernel's sink path)
          const bool row_on = q >= sink_row0;
          float pz[8], dz[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            pz[e] = row_on ? p[e] : 0.f;
            dz[e] = row_on ? ds[e] : 0.f;
          }
          uint16_t* Pt = ptile;
          uint16_t* St = ptile + 512;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int o = r32 * 16 + 8 * j + 4 * hf;
            *reinterpret_cast<u32x2*>(Pt + o) = u32x2{E::pack2(pz[4 * j], pz[4 * j + 1]), E::pack2(pz[4 * j + 2], pz[4 * j + 3])};
            *reinterpret_cast<u32x2*>(St + o) = u32x2{E::pack2(dz[4 * j], dz[4 * j + 1]), E::pack2(dz[4 * j + 2], dz[4 * j + 3])};
          }
          const int g4 = lane >> 4, i16 = lane & 15;
          const int pr = (8 * g4 + (i16 >> 2)) * 16 + 4 * (i16 & 3);
          const u32x2 pa0 = ds_read_tr16(Pt + pr), pa1 = ds_read_tr16(Pt + pr + 64);
          const u32x2 sa0 = ds_read_tr16(St + pr), sa1 = ds_read_tr16(St + pr + 64);
          const u32x4 pa = {pa0[0], pa0[1], pa1[0], pa1[1]}, sa = {sa0[0], sa0[1], sa1[0], sa1[1]};
#pragma unroll
          for (int nb = 0; nb < NB16; ++nb) {
            const int rr = 8 * g4 + (i16 >> 2), cc = 16 * nb + 4 * (i16 & 3);
            const u32x2 db0 = ds_read_tr16(Ds + swz_off<D>(rr, cc)), db1 = ds_read_tr16(Ds + swz_off<D>(rr + 4, cc));
            const u32x2 qb0 = ds_read_tr16(Qs + swz_off<D>(rr, cc)), qb1 = ds_read_tr16(Qs + swz_off<D>(rr + 4, cc));
            dvs[nb] = E::mfma16(pa, u32x4{db0[0], db0[1], db1[0], db1[1]}, dvs[nb]);
            dks[nb] = E::mfma16(sa, u32x4{qb0[0], qb0[1], qb1[0], qb1[1]}, dks[nb]);
          }
        }
      }
    }
    if (qt == qt0) {
      // the first tile's window halves (every wave's share): only the next tile's half and LSE,
      // issued at the top of this tile, may still be in flight
      if (has_next) wait_vm_lgkm0_barrier<2>();
      else wait_vm_lgkm0_barrier<1>();
    }
    refill_part();
    {
      // the row statistics for the dK/dV kernel (stored here, after the first tile's wait above)
      KArgs& A = args_fresh();
      if (hf == 0) {
        float* st = A.delta + ((int64_t(b) * A.Hq + h) * (A.Lp / 32) + qt) * 64;
        st[r32] = lse2;
        st[32 + r32] = ndelta;
      }
      if (A.sink_logits) {
        float v = q < L ? fast_exp2(fmaf(sink_logit, kLog2e, -lse2)) * delta : 0.f;
#pragma unroll
        for (int mm = 16; mm >= 1; mm >>= 1) v += __shfl_xor(v, mm);
        if (lane == 0) A.dsink_part[(int64_t(b) * A.Hq + h) * (A.Lp / 32) + qt] = -v;
      }
    }
    // the window halves, with the rest of the refill after the first two
    for (int j = hlo; j <= qt; ++j) {
      if (!wave_needs(32 * j, qw, L, W, S)) continue;
      float p[16], ds[16];
      half_step(ring + (j % kRing) * HALF, 32 * j, p, ds);
      if (refilled < 3) refill_part();
    }
    while (refilled < 3) refill_part();
    // the next tile's rows and K/V half have landed (waited before this tile's dQ stores, which
    // the next tile does not wait for)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (q < L) {
      KArgs& A = args_fresh();
      char* dqp = reinterpret_cast<char*>(A.dq) + 2 * slice_off(A.sdq, b, h, sq.row + q);
      const float scale = A.scale;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = acc[db][e] * scale;
        const int d0 = 32 * db + 16 * hf;
        st16(dqp + 2 * d0, pack8<E>(v));
        st16(dqp + 2 * (d0 + 8), pack8<E>(v + 8));
      }
    }
  }

  if constexpr (SINK) {
    // the waves' sink accumulators, summed in wave order through LDS (the ring: every wave is past
    // its last ring read after the barrier), into this unit's slot
    __syncthreads();
    KArgs& A = args_fresh();
    const int sr = A.srows;
    float* red = reinterpret_cast<float*>(ring);
    const int g4 = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int nb = 0; nb < NB16; ++nb)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int key = 4 * g4 + ii;
        if (key < sr) {
          red[((wave * 2 + 0) * sr + key) * D + 16 * nb + i16] = dks[nb][ii];
          red[((wave * 2 + 1) * sr + key) * D + 16 * nb + i16] = dvs[nb][ii];
        }
      }
    __syncthreads();
    const int n_out = 2 * sr * D;
    float* dst = A.dq_sink_part + int64_t(slot) * n_out;
    for (int x = tid; x < n_out; x += 512) {
      const int kind = x / (sr * D), rr = x % (sr * D);
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kSlideWaves; ++w) v += red[(w * 2 + kind) * sr * D + rr];
      dst[x] = v;
    }
  }
}

template <typename E>
static hipError_t launch_slide_e(const Args& a, hipStream_t stream) {
  const int per = a.vl_units ? a.vl_units : a.B * a.slide_ncu;  // units per (KV head, head group)
  const dim3 grid(unsigned(a.Hkv * (a.G / kSlideWaves) * per)), block(512);
  if (a.vl_units) {
    if (a.sink_dq) hipLaunchKernelGGL((bwd_dq_slide_kernel<E, true, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((bwd_dq_slide_kernel<E, false, true>), grid, block, 0, stream, a);
  } else {
    if (a.sink_dq) hipLaunchKernelGGL((bwd_dq_slide_kernel<E, true, false>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((bwd_dq_slide_kernel<E, false, false>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

hipError_t launch_bwd_dq_slide(const Args& a, int dtype, hipStream_t stream) {
  return dtype == 1 ? launch_slide_e<BF16>(a, stream) : launch_slide_e<F16>(a, stream);
}

}  // namespace fa
