// fa_bwd.hip - backward pass: dQ, dK, dV of masked attention, without atomics.
//
// Replaces FlashSWDAWithSink.backward's kernel (flash_attention_gpt_oss.py:183-338, 387-435)
// and the benchmark's split backward (_backward_dq_kernel / _backward_dkdv_kernel,
// benchmark_backward_speed.py:312-466).  The mathematics is the FA-2 backward
// (benchmark_backward_speed.py:132-141): with s = scale * q.k and P = exp(s - lse),
//     delta = rowsum(dO o O),  dP = dO V^T,  dS = P o (dP - delta),
//     dQ = scale * dS K,  dK = scale * dS^T Q,  dV = P^T dO,
// dK/dV summed over the query heads that share a KV head.
//
// Launches:
//  1. bwd_dq_kernel (query-major, same tiling as the forward): computes delta for its rows
//     (stored in the workspace) and dQ over the sink + window key blocks.  With at most 16 sink
//     keys in key block 0 (dq_sink_mode) it also accumulates those keys' dK/dV for the rows past
//     block 0's window, flushing fp32 partials to the workspace.
//  2. bwd_dkdv_kernel (key-major): a workgroup owns 64 keys of one KV head and sweeps the
//     (query head, 32-row query block) pairs that can see those keys, bounded by the window:
//     rows [k0, k0 + 63 + W).  Every sum is formed in a fixed order, so results are
//     deterministic.  Sink keys are also seen by every later row; outside dq_sink_mode those
//     rows are split into chunks of `chunk_rows` handled by extra workgroups of the same kernel
//     (the reference instead loops one program over all of L for a sink block,
//     benchmark_backward_speed.py:432-438).  In dq_sink_mode key block 0's workgroup adds the
//     dQ kernel's partials to its own when its sink keys' columns fit one pass of 256 threads.
//  3. bwd_sink_fold_kernel (when rows were chunked, or the in-kernel fold does not apply): adds
//     the sink rows' partial sums.
//  4. bwd_sink_logit_kernel (only with learned sink logits): adds the dQ kernel's per-row-block
//     partials of the sink logits' gradient.
#include <type_traits>

#include "fa_args.h"
#include "fa_common.h"

namespace fa {

// ---------------------------------------------------------------------------------------------
// dQ (query-major), persistent.  A tile is 32*wq rows x wh query heads of one KV group; a wave
// owns 32 rows of one head.  Per 32-key step, with S^T = K Q^T and dP^T = V dO^T in C layout
// (lane = query row), P and dS are per-lane elementwise, and dQ^T += K^T dS^T takes dS^T straight
// from registers while K^T is read transposed from the row-major K block in LDS.
//
// The grid is one wave of workgroups (resident together); every XCD owns a contiguous range of
// tiles (neighbouring tiles share K/V rows in that XCD's L2) and its workgroups walk it with the
// XCD's workgroup count as stride.  The rows of a workgroup's next tile (Q, dO, O, lse) are
// loaded while the current tile computes, so the row traffic overlaps the MFMA work.
//
// SINK (dq_sink_mode, S <= 16 sink keys): rows past key block 0's window see the sink keys only
// through the sink block, which this kernel visits for every tile anyway.  Their contributions to
// the sink keys' gradients, dV_s += P^T dO and dK_s += dS^T Q over keys [0, 16), accumulate here
// (v_mfma_f32_16x16x32, the tile's 32 rows as the reduction): P and dS of keys [0, 16) go through
// a per-wave LDS tile [32 rows][16 keys] to become the A operand, and dO / Q are read transposed
// from the wave's row-major stash tiles.  The accumulators are summed over the workgroup's waves
// and written once per run of tiles of one KV group (see the flush below), so the key-major
// kernel needs no workgroups for those rows.  (D = 128: each wave accumulates every wave's rows
// for a quarter of the head-dim columns instead; see SPLIT.)
// ---------------------------------------------------------------------------------------------
template <typename E, int D, bool SINK>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(const Args a) {
  constexpr int BN = 64;
  constexpr int KS = D / 16;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int BUF = 2 * BN * D;          // K, then V, both swizzled row-major [key][d]
  constexpr int CPB = BN * D / 8;          // 16-byte chunks per 64-key block of K (or V)
  constexpr int NK = (CPB + 255) / 256;    // chunks per thread
  constexpr bool ALL_ON = CPB >= 256;      // every thread loads a chunk of every tile
  constexpr int NX = 8;                    // XCDs: workgroup i runs on XCD i % 8
  constexpr int TILE = 32 * D;             // one 32-row tile, swizzled row-major [row][d]
  constexpr int STASH = 3 * TILE;          // per wave: the next tile's Q, dO, O tiles
  constexpr int NB16 = D / 16;             // 16-column blocks of the sink accumulators
  // the P / dS transposition tiles of the sink path: in the wave's O tile (read only for delta at
  // the start of a tile), or, for D = 16 where that tile is too small, in a region of their own
  constexpr int PT_EXTRA = (SINK && D < 32) ? 4 * 1024 : 0;
  // Small head dims (D <= 32): a key block's compute is short next to the latency of fetching the
  // next one, so (as in the forward) every block of a tile, up to NBUF at a time, is fetched at
  // once by LDS DMA into a buffer of its own and the blocks are then computed back to back; the
  // first tile's rows come in the same round trip.  Wider heads double-buffer (see KDMA).
  constexpr bool PRE = D <= 32;
  // D >= 64: key blocks by DMA into two buffers, one block ahead (16 registers fewer than staging
  // them through registers at D = 64, 32 at D = 128; c3 dQ 867 -> 839 us).
  constexpr bool KDMA = D >= 64;
  // D = 128 with sink rows: the sink keys' accumulators are split over the 4 waves by head-dim
  // columns (16 registers a wave instead of 64), each wave taking every wave's rows for its 32
  // columns (sink_split below), which leaves the D = 128 key loop (see compute_block) the
  // registers it needs without spilling to scratch memory.
  constexpr bool SPLIT = SINK && D == 128;
  constexpr int NSA = SPLIT ? D / 64 : D / 16;  // 16-column blocks of the sink accumulators per wave
  constexpr int NBUF = PRE ? 32768 / (2 * BUF) : 2;  // 32 KiB of K/V blocks
  __shared__ __attribute__((aligned(16))) uint16_t lds[NBUF * BUF + 4 * STASH + PT_EXTRA];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform in a scalar register, so that per-wave rows, heads and buffer descriptors stay
  // scalar (no per-lane copies, no waterfall loops around buffer loads)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int W = a.W, S = a.S;

  // this workgroup's tiles: its XCD's range [t_lo, t_hi), walked in rounds of wgs_x consecutive
  // tiles, one per workgroup.  Without sink rows, round r gives workgroup pos the tile pos for even
  // r and wgs_x - 1 - pos for odd r, which evens out the work of causal tiles (it grows with the
  // row); with sink rows the order stays pos in every round (a stride of wgs_x), which the runs of
  // sink partials and bwd_sink_fold_kernel rely on.
  const int groups = a.B * a.Hq / a.wh;
  const int n_tiles = a.n_qtiles * groups;
  const int xcd = blockIdx.x % NX, pos = blockIdx.x / NX, wgs_x = gridDim.x / NX;
  const int per = n_tiles / NX, rem = n_tiles % NX;
  const int t_lo = xcd * per + min(xcd, rem), t_hi = t_lo + per + (xcd < rem ? 1 : 0);
  // tiles per (batch, KV head): n_qtiles row tiles of each of the G / wh head groups
  const int tiles_per_kv = a.n_qtiles * (a.G / a.wh);

  // tile -> (b, KV head, this wave's head hw, first row qw, the sequence's length L and first row)
  struct TileIdx {
    int b, kvh, hw, q0, qw, L;
    int64_t row;
  };
  // Tile order, slowest first: KV head, batch, head group of the KV head, row tile -- the tiles of
  // one (batch, KV head) are contiguous, tiles_per_kv of them starting at (b + B kvh) tiles_per_kv.
  // The KV head is outermost so that the XCD ranges split over KV heads before they split over
  // sequences: with at least 8 KV heads every XCD gets the same sequences, so the work stays even
  // when the sequences of a variable-length batch differ in length.
  auto decode = [&](int tile) {
    KArgs& A = args_fresh();
    TileIdx t;
    const int qt = tile % A.n_qtiles, hg = tile / A.n_qtiles;
    const int gpk = A.G / A.wh;  // head groups per KV head
    const int bk = hg / gpk;
    t.b = bk % A.B;
    t.kvh = bk / A.B;
    const Seq sq = seq_of(A, t.b);
    t.L = sq.L;
    t.row = sq.row;
    const int h0 = t.kvh * A.G + (hg % gpk) * A.wh;
    t.q0 = qt * 32 * A.wq;
    t.qw = t.q0 + 32 * (wave % A.wq);
    t.hw = h0 + wave / A.wq;
    return t;
  };

  // The rows of a tile for this wave: Q, dO and O go by LDS DMA into the wave's own stash as
  // swizzled row-major [32][D] tiles (DMA instruction p, lane l fills 16-byte position 64p + l, so
  // it loads the global chunk that the swizzle places there), where they occupy no registers
  // while the current tile computes; the row's lse goes to a register.  Buffer resources over the
  // sequence's rows [0, L) of the head: rows past L read as zero.
  uint16_t* stash = lds + NBUF * BUF + wave * STASH;
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  auto stash_rows = [&](const TileIdx& t) {
    KArgs& A = args_fresh();
    const rsrc_t rq = make_rsrc(reinterpret_cast<const char*>(A.q) + 2 * slice_off(A.sq, t.b, t.hw, t.row), span_bytes(t.L, A.sq[2], D));
    const rsrc_t rd = make_rsrc(reinterpret_cast<const char*>(A.dout) + 2 * slice_off(A.sdo, t.b, t.hw, t.row), span_bytes(t.L, A.sdo[2], D));
    const rsrc_t ro = make_rsrc(reinterpret_cast<const char*>(A.o) + 2 * slice_off(A.so, t.b, t.hw, t.row), span_bytes(t.L, A.so[2], D));
    const int64_t sq2 = A.sq[2], sdo2 = A.sdo[2], so2 = A.so[2];
#pragma unroll
    for (int p = 0; p < KS; ++p) {
      const int tr = (64 * p + lane) / CPR;  // tile row of this lane's 16-byte position
      const int col = 8 * (((64 * p + lane) % CPR) ^ swz<D>(tr));
      const int64_t row = t.qw + tr;
      buf_dma16(rq, stash + 0 * TILE + 512 * p, uint32_t((row * sq2 + col) * 2));
      buf_dma16(rd, stash + 1 * TILE + 512 * p, uint32_t((row * sdo2 + col) * 2));
      buf_dma16(ro, stash + 2 * TILE + 512 * p, uint32_t((row * so2 + col) * 2));
    }
  };
  auto load_lse = [&](const TileIdx& t) {
    KArgs& A = args_fresh();
    const rsrc_t rl = make_rsrc(A.lse + slice_off(A.slse, t.b, t.hw, t.row), span_f32(t.L, A.slse[2]));
    return buf_ldf(rl, uint32_t(int64_t(t.qw + r32) * A.slse[2] * 4));
  };

  // K/V staging offsets (the same for every tile)
  uint32_t off_k[NK], off_v[NK];
  int off_l[NK];
#pragma unroll
  for (int it = 0; it < NK; ++it) {
    const int c = tid + 256 * it;
    const int row = c / (D / 8), col = c % (D / 8);
    off_k[it] = uint32_t((int64_t(row) * a.sk[2] + 8 * col) * 2);
    off_v[it] = uint32_t((int64_t(row) * a.sv[2] + 8 * col) * 2);
    off_l[it] = swz_off<D>(row, 8 * col);
  }
  const uint32_t bk = uint32_t(2 * a.sk[2]), bv = uint32_t(2 * a.sv[2]);  // bytes per key row

  // sink accumulators: lane l holds key 4(l/16) + i, head-dim column 16 nb + l % 16 (SPLIT: column
  // 16 (NSA wave + nb) + l % 16)
  f32x4 dks[SINK ? NSA : 1], dvs[SINK ? NSA : 1];
  if constexpr (SINK) {
#pragma unroll
    for (int nb = 0; nb < NSA; ++nb) {
      dks[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
      dvs[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  uint16_t* ptile = SINK ? (D >= 32 ? stash + 2 * TILE : lds + NBUF * BUF + 4 * STASH + wave * 1024) : nullptr;

  auto tile_of = [&](int r) { return t_lo + r * wgs_x + ((!SINK && (r & 1)) ? wgs_x - 1 - pos : pos); };
  const int first_tile = tile_of(0);
  int run_first = first_tile;  // first tile of the current run of tiles of one (batch, KV head)
  float lse_next = 0.f;
  if (!PRE && first_tile < t_hi) {
    const TileIdx t0 = decode(first_tile);
    stash_rows(t0);
    lse_next = load_lse(t0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  // (A round counter rather than the forward's step: with the step, the D = 128 variant with sink
  // rows, at its register limit, waited for a load one block earlier, 3% more at c5.)
  for (int r = 0; t_lo + r * wgs_x < t_hi; ++r) {
    const int tile = tile_of(r);
    if (tile >= t_hi) continue;  // the last round is short
    // the workgroup's next tile (the round after a short last round does not exist)
    const int next_tile = tile_of(r + 1);
    const bool has_next = next_tile < t_hi;
    const TileIdx t = decode(tile);
    const int qw = t.qw, q = qw + r32, L = t.L;
    const bool wave_active = qw < L;

    const QPlan plan = qplan(t.q0, 32 * a.wq, L, W, S);
    KArgs& Akv = args_fresh();
    const rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(Akv.k) + 2 * slice_off(Akv.sk, t.b, t.kvh, t.row), span_bytes(L, Akv.sk[2], D));
    const rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(Akv.v) + 2 * slice_off(Akv.sv, t.b, t.kvh, t.row), span_bytes(L, Akv.sv[2], D));
    // PRE: DMA of a 64-key block into buffer j -- the block's K and V tiles are CPB 16-byte chunks
    // each, 2 CPB / 64 instructions of 64 lanes; wave w issues instructions [w NIW, (w + 1) NIW),
    // and lane l of instruction p (of K or V) loads the chunk that the swizzle places at position
    // 64 p + l (as the forward's)
    constexpr int IPT = CPB / 64;
    constexpr int NIW = (PRE || KDMA) ? 2 * IPT / 4 : 1;
    static_assert(!(PRE || KDMA) || (NIW >= 1 && 2 * IPT == 4 * NIW), "whole DMA instructions per wave");
    auto dma_block = [&](int kb, int j) {
#pragma unroll
      for (int n = 0; n < NIW; ++n) {
        const int ii = wave * NIW + n, is_v = ii >= IPT, pi = is_v ? ii - IPT : ii;
        const int dpos = 64 * pi + lane, row = dpos / CPR, col = (dpos % CPR) ^ swz<D>(row);
        uint16_t* dst = lds + j * BUF + (is_v ? BN * D : 0) + 512 * pi;
        const uint32_t off = uint32_t(int64_t(kb + row) * (is_v ? bv : bk)) + 16u * uint32_t(col);
        if (is_v) buf_dma16(rv, dst, off);
        else buf_dma16(rk, dst, off);
      }
    };
    if constexpr (PRE) {
      const int ng = min(NBUF, plan.nb);
      for (int j = 0; j < ng; ++j) dma_block(qplan_block(plan, j), j);
      if (tile == first_tile) {  // the first tile's rows, in the same round trip as its blocks
        stash_rows(t);
        lse_next = load_lse(t);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }

    // Row operands and row statistics, from the stash (this wave's own DMA, complete by now:
    // see the wait after the key loop).  delta = rowsum(dO o O) is stored for the dK/dV kernel;
    // the dP accumulator of every key tile starts from -delta, so dS = P * acc.
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
    const float lse2 = q < L ? lse_next * kLog2e : __builtin_inff();
    {
      KArgs& A = args_fresh();
      // the row statistics of the dK/dV kernel: per 32-row block, lse * log2(e) for the 32 rows,
      // then -delta (rows past L: +inf and 0, so that their P and dS there are exactly 0)
      if (hf == 0 && wave_active) {  // (an active wave's rows are all < Lp)
        float* st = A.delta + ((int64_t(t.b) * A.Hq + t.hw) * (A.Lp / 32) + qw / 32) * 64;
        st[r32] = lse2;
        st[32 + r32] = ndelta;
      }
      if (A.sink_logits && wave_active) {
        // learned sink: d sink = -sum over rows of P_sink * delta, P_sink = 2^(sink*log2e - lse2);
        // one partial per 32-row block, summed in a fixed order by bwd_sink_logit_kernel
        float v = q < L ? fast_exp2(A.sink_logits[t.hw] * kLog2e - lse2) * delta : 0.f;
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m);
        if (lane == 0) A.dsink_part[(int64_t(t.b) * A.Hq + t.hw) * (A.Lp / 32) + qw / 32] = -v;
      }
    }
    // this wave's rows add to the sink keys' gradients (rows past key block 0's window)
    const int sink_row0 = dq_sink_row0(L, W);
    const bool sink_rows = SINK && wave_active && qw + 31 >= sink_row0;

    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

    u32x4 kreg[NK], vreg[NK];
    auto gload = [&](int kb) {
#pragma unroll
      for (int it = 0; it < NK; ++it) {
        if (ALL_ON || tid + 256 * it < CPB) {
          kreg[it] = buf_ld16(rk, off_k[it] + uint32_t(kb) * bk);
          vreg[it] = buf_ld16(rv, off_v[it] + uint32_t(kb) * bv);
        }
      }
    };
    auto sstore = [&](int buf) {
      uint16_t* Kl = lds + buf * BUF;
      uint16_t* Vl = Kl + BN * D;
#pragma unroll
      for (int it = 0; it < NK; ++it) {
        if (ALL_ON || tid + 256 * it < CPB) {
          st16(Kl + off_l[it], kreg[it]);
          st16(Vl + off_l[it], vreg[it]);
        }
      }
    };
    // the next tile's rows into the stash, once this tile's have been read out of it (and, on
    // the sink path, after the transposed reads of its Q and dO tiles in key block 0)
    auto refill = [&]() {
      if (has_next) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const TileIdx tn = decode(next_tile);
        stash_rows(tn);
        lse_next = load_lse(tn);
      }
    };

    // The sink keys' dV_s += P^T dO and dK_s += dS^T Q of one wave's 32 rows: P and dS from the
    // [32 rows][16 keys] tiles Pt / St, dO and Q from the stash tiles Dt / Qt, into the accumulators'
    // NSA 16-column blocks starting at column block nb0.
    auto sink_products = [&](const uint16_t* Pt, const uint16_t* St, const uint16_t* Qt, const uint16_t* Dt, int nb0) {
      // A operands P^T / dS^T (16 keys x 32 rows): lane l gets key l % 16, rows 8(l/16) + 0..7, by
      // two transposing reads of 4 rows each
      const int g4 = lane >> 4, i16 = lane & 15;
      const int pr = (8 * g4 + (i16 >> 2)) * 16 + 4 * (i16 & 3);
      const u32x2 pa0 = ds_read_tr16(Pt + pr), pa1 = ds_read_tr16(Pt + pr + 64);
      const u32x2 sa0 = ds_read_tr16(St + pr), sa1 = ds_read_tr16(St + pr + 64);
      const u32x4 pa = {pa0[0], pa0[1], pa1[0], pa1[1]}, sa = {sa0[0], sa0[1], sa1[0], sa1[1]};
#pragma unroll
      for (int nb = 0; nb < NSA; ++nb) {
        // B operands dO / Q (32 rows x 16 columns): lane l gets column 16 (nb0 + nb) + l % 16 of the
        // same rows, read transposed from the stash tiles
        const int rr = 8 * g4 + (i16 >> 2), cc = 16 * (nb0 + nb) + 4 * (i16 & 3);
        const u32x2 db0 = ds_read_tr16(Dt + swz_off<D>(rr, cc)), db1 = ds_read_tr16(Dt + swz_off<D>(rr + 4, cc));
        const u32x2 qb0 = ds_read_tr16(Qt + swz_off<D>(rr, cc)), qb1 = ds_read_tr16(Qt + swz_off<D>(rr + 4, cc));
        dvs[nb] = E::mfma16(pa, u32x4{db0[0], db0[1], db1[0], db1[1]}, dvs[nb]);
        dks[nb] = E::mfma16(sa, u32x4{qb0[0], qb0[1], qb1[0], qb1[1]}, dks[nb]);
      }
    };
    // SPLIT, after key block 0 of a tile with sink rows (every wave, whatever its rows): once every
    // wave has written its P / dS tiles, each wave adds the products of every wave's rows (in wave
    // order) to its own NSA column blocks; the barrier after them precedes the refill of the stashes.
    auto sink_split = [&]() {
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int qu = t.q0 + 32 * (u % a.wq);  // wave u's rows
        if (qu < L && qu + 31 >= sink_row0) {
          const uint16_t* su = lds + NBUF * BUF + u * STASH;
          sink_products(su + 2 * TILE, su + 2 * TILE + 512, su, su + TILE, NSA * wave);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    // does any wave of the tile have sink rows (the condition of sink_split, uniform over the
    // workgroup)?
    const bool tile_sink = SPLIT && t.q0 < L && t.q0 + 32 * a.wq - 1 >= sink_row0;

    // one key block [kb, kb + 64) from the K tile at Kl (V follows it)
    auto compute_block = [&](int kb, const uint16_t* Kl) {
      if (wave_active) {
        const uint16_t* Vl = Kl + BN * D;
        if constexpr (D == 128) {
          // One wave per SIMD: when both 32-key halves of the block are unmasked (and the sink path
          // does not need the first half's P and dS), both halves' score products are issued before
          // either half's elementwise work, in one basic block, so that the second half's products
          // run under the first half's exponentials.  The same operations per accumulator, in the
          // same order, as the loop below.  With the DMA staging, the split sink accumulators and
          // the one-chain masked path: c5 dQ 388 -> 367 us, and 347 -> 319 us without sink keys.
          if (tile_full(kb, qw, W, S) && tile_full(kb + 32, qw, W, S) && !(SINK && kb == 0 && sink_rows)) {
            f32x16 s2[2], dp2[2];
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
              u32x4 kf[KS], vf[KS];
#pragma unroll
              for (int ks = 0; ks < KS; ++ks) {
                const int off = swz_off<D>(32 * sb + r32, hf * (D / 2) + 8 * ks);
                kf[ks] = *reinterpret_cast<const u32x4*>(Kl + off);
                vf[ks] = *reinterpret_cast<const u32x4*>(Vl + off);
              }
              f32x16 d0;
#pragma unroll
              for (int e = 0; e < 16; ++e) d0[e] = ndelta;
#pragma unroll
              for (int ks = 0; ks < KS; ++ks) {
                s2[sb] = E::mfma(kf[ks], qf[ks], ks == 0 ? f32x16{} : s2[sb]);
                dp2[sb] = E::mfma(vf[ks], dof[ks], ks == 0 ? d0 : dp2[sb]);
              }
            }
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
              float ds[16];
#pragma unroll
              for (int e = 0; e < 16; ++e) ds[e] = fast_exp2(fmaf(s2[sb][e], a.c, -lse2)) * dp2[sb][e];
              const u32x4 d0 = pack8<E>(ds), d1 = pack8<E>(ds + 8);
#pragma unroll
              for (int db = 0; db < DB; ++db) {
                acc[db] = E::mfma(tr_frag_swz<D>(Kl, 32 * sb, 32 * db, D), d0, acc[db]);
                acc[db] = E::mfma(tr_frag_swz<D>(Kl, 32 * sb + 16, 32 * db, D), d1, acc[db]);
              }
            }
            return;
          }
        }
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const int ks0 = kb + 32 * sb;
          if (!wave_needs(ks0, qw, L, W, S)) continue;
          // S^T = K Q^T and dP^T - delta = V dO^T - delta.  Masked tiles start S^T from an
          // additive bias, 0 (allowed) or -inf (masked), so P is exactly 0 there; the test is
          // the forward's: register e holds key ks0 + 4hf + off(e), allowed = (dq0 - off) < lim.
          u32x4 kf[KS], vf[KS];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const int off = swz_off<D>(32 * sb + r32, hf * (D / 2) + 8 * ks);
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
          // (D = 128: full blocks take the path above; here the mask's bias is formed for every
          // tile -- 0 throughout when it is full -- so that one chain of score products is emitted
          // and the K/V operands stay next to it)
          if (D != 128 && tile_full(ks0, qw, W, S)) {
            qk(f32x16{});
          } else {
            f32x16 bias;
            const int dq0 = q - ks0 - 4 * hf;
            if (ks0 >= S || ks0 + 32 <= S) {  // one limit for all 32 keys
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
          // dQ^T += K^T dS^T: K^T read transposed from the row-major K block, keys in the row
          // order of the dS^T C tile
          float p[16], ds[16];
          // D = 64: P, dS and the dQ products at a higher issue priority than the score products
          // of the other workgroup's wave on the SIMD (c3 dQ 864 -> 828 us; D = 128, one wave per
          // SIMD, was 4% slower with it, D = 16 unchanged)
          if constexpr (D == 64) __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            p[e] = fast_exp2(fmaf(s[e], a.c, -lse2));
            ds[e] = p[e] * dp[e];
          }
          const u32x4 d0 = pack8<E>(ds), d1 = pack8<E>(ds + 8);
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            acc[db] = E::mfma(tr_frag_swz<D>(Kl, 32 * sb, 32 * db, D), d0, acc[db]);
            acc[db] = E::mfma(tr_frag_swz<D>(Kl, 32 * sb + 16, 32 * db, D), d1, acc[db]);
          }
          if constexpr (D == 64) __builtin_amdgcn_s_setprio(0);
          if constexpr (SINK) {
            if (ks0 == 0 && sink_rows) {
              // P and dS of keys [0, 16) (registers 0..7: keys 4hf + 0..3 and 8 + 4hf + 0..3 of
              // row q), rows before sink_row0 zeroed, into the [32 rows][16 keys] tiles
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
              if constexpr (!SPLIT) sink_products(Pt, St, Qs, Ds, 0);  // (SPLIT: in sink_split)
            }
          }
        }
      }
    };

    if constexpr (PRE) {
      for (int g0 = 0; g0 < plan.nb; g0 += NBUF) {
        const int ng = min(NBUF, plan.nb - g0);
        if (g0 > 0)
          for (int j = 0; j < ng; ++j) dma_block(qplan_block(plan, g0 + j), j);
        // the blocks have landed everywhere (the next tile's rows may be in flight)
        if (g0 == 0 && !SINK) {
          refill();
          if (has_next) wait_vm_lgkm0_barrier<3 * KS + 1>();
          else wait_vm_lgkm0_barrier<0>();
        } else {
          wait_vm_lgkm0_barrier<0>();
        }
        for (int j = 0; j < ng; ++j) {
          compute_block(qplan_block(plan, g0 + j), lds + j * BUF);
          if (SINK && g0 == 0 && j == 0) refill();
        }
        __syncthreads();  // before the buffers are refilled
      }
    } else if constexpr (KDMA) {
      // block i in buffer i & 1; block i + 1's DMA is issued before block i computes (its buffer was
      // last read by block i - 1, behind the barrier that ended it) and waited for after it.  The
      // next tile's rows (refill, 3 KS + 1 loads) are issued after block 1's DMA and may stay in
      // flight past block 0's wait; later waits find them landed.
      // D = 128 without sink rows issues the refill with block 0's DMA, one block earlier (c5
      // without sink keys: dQ 325 -> 314 us; D = 64 measured 0.6% slower).
      constexpr bool EARLY = !SINK && D == 128;
      if (plan.nb > 0) {
        dma_block(qplan_block(plan, 0), 0);
        if (EARLY) refill();
        if (EARLY && has_next) wait_vm_lgkm0_barrier<3 * KS + 1>();
        else wait_vm_lgkm0_barrier<0>();
      }
      for (int i = 0; i < plan.nb; ++i) {
        const bool more = i + 1 < plan.nb;
        if (more) dma_block(qplan_block(plan, i + 1), (i + 1) & 1);
        if (!SINK && !EARLY && i == 0) refill();
        compute_block(qplan_block(plan, i), lds + (i & 1) * BUF);
        if (SPLIT && i == 0 && tile_sink && qplan_block(plan, 0) == 0) sink_split();
        if (SINK && i == 0) refill();
        if (!EARLY && i == 0 && has_next) wait_vm_lgkm0_barrier<3 * KS + 1>();
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
        if (!SINK && i == 0) refill();
        compute_block(qplan_block(plan, i), lds + (i & 1) * BUF);
        if (SPLIT && i == 0 && tile_sink && qplan_block(plan, 0) == 0) sink_split();
        if (SINK && i == 0) refill();
        if (more) sstore((i + 1) & 1);
        __syncthreads();
      }
    }
    if (plan.nb == 0) refill();  // no key block (cannot happen for valid masks; kept for safety)
    // the next tile's stash has landed (waited here, before this tile's dQ stores, which would
    // otherwise also be waited for)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    if (wave_active && q < L) {
      KArgs& A = args_fresh();
      char* dqp = reinterpret_cast<char*>(A.dq) + 2 * slice_off(A.sdq, t.b, t.hw, t.row + q);
      const float scale = A.scale;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        if (D == 16 && hf == 1) continue;
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = acc[db][e] * scale;
        const int d0 = 32 * db + (D >= 32 ? 16 * hf : 0);
        st16(dqp + 2 * d0, pack8<E>(v));
        st16(dqp + 2 * (d0 + 8), pack8<E>(v + 8));
      }
    }

    if constexpr (SINK) {
      // Flush at the end of a run of tiles of one (batch, KV head): the waves' accumulators are
      // summed in LDS (the K/V buffers: every wave has passed the key loop's last barrier, and
      // the next tile stages K/V only after the barrier below) in wave order and written to the
      // slot of the run's first tile.  A workgroup has at most one run per (batch, KV head), and
      // the runs of one XCD start at the first wgs_x tiles of its share of that (batch, KV head),
      // which is how bwd_sink_fold_kernel finds the slots.
      const bool flush = !has_next || next_tile / tiles_per_kv != tile / tiles_per_kv;
      if constexpr (SPLIT) {
        // each wave holds the whole workgroup's sums for its own columns: written as they are
        if (flush) {
          KArgs& A = args_fresh();
          const int sr = A.srows;
          float* slot = A.dq_sink_part + int64_t(run_first) * (2 * sr * D);
          run_first = next_tile;
          const int g4 = lane >> 4, i16 = lane & 15;
#pragma unroll
          for (int nb = 0; nb < NSA; ++nb) {
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const int key = 4 * g4 + ii;
              if (key < sr) {
                slot[(0 * sr + key) * D + 16 * (NSA * wave + nb) + i16] = dks[nb][ii];
                slot[(1 * sr + key) * D + 16 * (NSA * wave + nb) + i16] = dvs[nb][ii];
              }
            }
            dks[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
            dvs[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
      } else if (flush) {
        KArgs& A = args_fresh();
        const int sr = A.srows;
        float* red = reinterpret_cast<float*>(lds);
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
        float* slot = A.dq_sink_part + int64_t(run_first) * n_out;
        run_first = next_tile;
        for (int x = tid; x < n_out; x += 256) {
          const int kind = x / (sr * D), rest = x % (sr * D);
          float v = 0.f;
#pragma unroll
          for (int w = 0; w < 4; ++w) v += red[(w * 2 + kind) * sr * D + rest];
          slot[x] = v;
        }
        __syncthreads();
#pragma unroll
        for (int nb = 0; nb < NB16; ++nb) {
          dks[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dvs[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
}

// K^T / V^T operands of a dK/dV wave (B of S = Q K^T and dP = dO V^T): lane (key, hf), head-dim
// slice [hf D/2 + 8ks, +8), through buffer resources over the KV head's rows [0, L), so keys >= L
// read as zero with no per-lane select -- nothing uses the registers, and so nothing waits for
// them, until kv_operands_ready.  (K keeps its sign: the kernels take a negative softmax scale
// in the exponent's factor.)
template <int D>
__device__ __forceinline__ void load_kv_operands(const Args& a, int b, int kvh, const Seq& sq, int key,
                                                 u32x4 (&kf)[D / 16], u32x4 (&vf)[D / 16]) {
  const int hf = (threadIdx.x >> 5) & 1;
  const rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(a.k) + 2 * slice_off(a.sk, b, kvh, sq.row),
                              span_bytes(sq.L, a.sk[2], D));
  const rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(a.v) + 2 * slice_off(a.sv, b, kvh, sq.row),
                              span_bytes(sq.L, a.sv[2], D));
  const uint32_t ko = uint32_t(int64_t(key) * a.sk[2] * 2), vo = uint32_t(int64_t(key) * a.sv[2] * 2);
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const uint32_t d2 = uint32_t(2 * (hf * (D / 2) + 8 * ks));
    kf[ks] = buf_ld16(rk, ko + d2);
    vf[ks] = buf_ld16(rv, vo + d2);
  }
}
// Where the K/V operand loads must have landed: an empty asm statement that reads and rewrites
// the registers, so the compiler's own wait for them goes here -- after the caller's first DMA
// issues, which stay in flight -- and not before the first product inside the step loop, where it
// would be repeated every step and wait for the DMA of later steps too.
template <int KS>
__device__ __forceinline__ void kv_operands_ready(u32x4 (&kf)[KS], u32x4 (&vf)[KS]) {
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kf[ks]), "+v"(vf[ks]));
}

// dV^T += dO^T P and dK^T += Q^T dS over the DB 32-column blocks of head dim, for one 32-row item:
// P and dS as B operands (pb, sb: rows 0-15 and 16-31), dO^T / Q^T read transposed from the
// swizzled row-major tiles Qt and Dt.
template <typename E, int D, int DB>
__device__ __forceinline__ void dkdv_products(const uint16_t* Qt, const uint16_t* Dt, const u32x4 (&pb)[2],
                                              const u32x4 (&sb)[2], f32x16 (&dv)[DB], f32x16 (&dk)[DB]) {
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const u32x4 dt = tr_frag_swz<D>(Dt, 16 * t, 32 * db, D);
      const u32x4 qt = tr_frag_swz<D>(Qt, 16 * t, 32 * db, D);
      dv[db] = E::mfma(dt, pb[t], dv[db]);
      dk[db] = E::mfma(qt, sb[t], dk[db]);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dK / dV (key-major).  A workgroup owns 64 keys of one KV head; wave (kh, hh) = (wave & 1,
// wave >> 1) owns the 32-key half kh and takes head slot hh of every step.  A step stages two
// (query head, 32-row block) items -- Q and dO rows plus their lse * log2(e) and -delta -- in LDS,
// shared by the two waves of each slot; they arrive by DMA, issued a few steps ahead into a ring
// of LDS stages.  Per item and wave: S = Q K^T and dP = dO V^T in C layout (lane = key column, 16
// query rows per lane), P and dS elementwise, then dV^T += dO^T P and dK^T += Q^T dS with P/dS
// straight from registers and dO^T/Q^T read transposed from the row-major tiles
// (ds_read_b64_tr_b16).  The two head slots' partial sums are added in LDS at the end.
//
// Sink keys: for the first `nsp` blocks the rows past the window are handled by chunk
// workgroups; every workgroup of such a block writes the fp32 partial sums of its sink rows to
// its own slot of the workspace, and bwd_sink_fold_kernel adds the slots in a fixed order.
// ---------------------------------------------------------------------------------------------
// Adds up the sink keys' dK/dV partials (defined with bwd_sink_fold_kernel below).
template <typename E, int D>
__device__ void fold_sink_keys(int b, int kvh, int nk, const Seq& sq, float* smem);

// The dK/dV kernel's LDS stages (see its staging).  KVL (D = 64 only): the K and V tiles of the
// workgroup's 64 keys sit in LDS as well, and the score products read their B operands from there
// every step instead of holding them in 32 registers; with two stages that leaves 160 VGPRs and
// 49 KB of LDS, three workgroups per CU instead of two.
__host__ __device__ constexpr int dkdv_stages(int D, bool kvl) { return D == 128 ? 3 : kvl ? 2 : 4; }
// 16-bit elements of the dK/dV kernel's LDS: the stages of two items each (Q and dO tiles, 32
// rows, and 128 elements of row statistics per item) and with KVL the K/V tiles, or the fp32
// partials of the head-slot sum if larger.
__host__ __device__ constexpr int dkdv_lds_elems(int D, bool kvl) {
  const int stages = dkdv_stages(D, kvl) * 2 * (2 * 32 * D + 128) + (kvl ? 4 * 32 * D : 0);
  const int red = 2 * 2 * 2 * (D >= 32 ? D / 32 : 1) * 16 * 64;
  return stages > red ? stages : red;
}

// Does key block 0's workgroup fold the sink keys itself (dq_sink_mode; the dQ kernel's run list
// and the chunk sums fit the kernel's LDS)?  Otherwise bwd_sink_fold_kernel does it after the
// dK/dV kernel.  Up to 256 (sink key, column) pairs the workgroup's threads split the runs as well
// (fold_sink_keys); up to 2048 each thread sums whole chunks of four columns over every run.
__host__ __device__ inline bool dkdv_folds_in_kernel(const Args& a, int D, bool kvl) {
  return a.sink_dq && (a.S < kKvKeys ? a.S : kKvKeys) * D <= 2048 &&
         ((a.dq_wgs + 3) & ~3) + 4 * 256 <= dkdv_lds_elems(D, kvl) / 2;
}

// D = 16 keeps four waves per SIMD (at most 128 VGPRs), D = 64 with KVL three (168); the wider
// head dims need more registers.
template <typename E, int D, bool KVL = false>
__global__ __launch_bounds__(256, D == 16 ? 4 : KVL ? 3 : 1) void bwd_dkdv_kernel(const Args a) {
  constexpr int KS = D / 16;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int TILE = 32 * D;               // 32 rows of Q or dO, swizzled row-major
  constexpr int SLOT = 2 * TILE + 128;       // Q, dO, then lse2[32] and -delta[32] as fp32
  constexpr int STAGE = 2 * SLOT;            // two items per step
  constexpr int NSTG = dkdv_stages(D, KVL);  // LDS stages: see the staging below
  static_assert(!KVL || D == 64, "K/V operands from LDS: D = 64 only");
  constexpr int CPR = D / 8;                 // 16-byte chunks per row
  __shared__ __attribute__((aligned(16))) uint16_t lds[dkdv_lds_elems(D, KVL)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int kh = wave & 1, hh = wave >> 1;
  const int W = a.W, S = a.S, G = a.G;

  // Workgroups come in groups per (b, KV head): the n_kblocks regular ones, then the sink
  // chunks.  A group's workgroups land on one XCD (they share its L2), and the short chunk
  // workgroups run last, filling the slots that the regular ones leave.
  const int per_group = a.n_kblocks + a.nsp * a.n_chunks;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  // groups in (KV head, batch) order, the KV head outermost: the XCDs then split over KV heads
  // before sequences, which keeps their work even for sequences of different lengths.  A packed
  // batch hands out only the key blocks with keys: per KV head, each sequence's blocks
  // (varlen_nth), then the sequences' chunk workgroups.
  int kvh, b, r;
  if (a.vl_kblocks) {
    const int n_cw = a.nsp * a.n_chunks;
    const int per_kv = a.vl_kblocks + a.B * n_cw;
    kvh = id / per_kv;
    const int p = id % per_kv;
    if (p < a.vl_kblocks) {
      if (!varlen_nth(a, p, a.vl_kblocks, kKvKeys, 1, b, r)) return;
    } else {
      b = (p - a.vl_kblocks) / n_cw;
      r = a.n_kblocks + (p - a.vl_kblocks) % n_cw;
    }
  } else {
    const int grp = id / per_group;
    r = id % per_group;
    kvh = grp / a.B;
    b = grp % a.B;
  }
  const Seq sq = seq_of(a, b);
  const int L = sq.L;
  int kblk, chunk = -1, qlo, qhi;
  if (r < a.n_kblocks) {
    kblk = r;
    qlo = kKvKeys * kblk;
    qhi = kv_window_end(kblk, L, W);
  } else {
    const int t = r - a.n_kblocks;
    kblk = t % a.nsp;
    chunk = t / a.nsp;
    qlo = kv_chunk_lo(kblk, chunk, a.chunk_rows, L, W);
    qhi = kv_chunk_hi(kblk, chunk, a.chunk_rows, L, W);
  }
  // a key block past the end of its sequence (variable-length batches) has nothing to do; the
  // sink fold reads no slot of it
  if (kKvKeys * kblk >= L) return;
  const bool is_chunk = chunk >= 0;
  const bool partial_block = kblk < a.nsp;
  const int ks0 = kKvKeys * kblk + 32 * kh;  // this wave's keys
  const int key = ks0 + r32;
  const bool wave_on = ks0 < L && (!is_chunk || ks0 < S);
  const int wqlo = is_chunk ? qlo : max(qlo, ks0), wqhi = qhi;

  // K^T / V^T operands, waited for after the first DMA issues (load_kv_operands), or (KVL) the
  // workgroup's K and V tiles by DMA into LDS: wave w loads tile w (K of half 0, V of half 0, K of
  // half 1, V of half 1), swizzled row-major like the Q / dO tiles
  u32x4 kf[KVL ? 1 : KS], vf[KVL ? 1 : KS];
  uint16_t* const kvl = lds + NSTG * STAGE;
  if constexpr (KVL) {
    const bool tv = wave & 1;
    const int64_t rs = tv ? a.sv[2] : a.sk[2];
    const rsrc_t r = tv ? make_rsrc(reinterpret_cast<const char*>(a.v) + 2 * slice_off(a.sv, b, kvh, sq.row), span_bytes(L, a.sv[2], D))
                        : make_rsrc(reinterpret_cast<const char*>(a.k) + 2 * slice_off(a.sk, b, kvh, sq.row), span_bytes(L, a.sk[2], D));
    const int k0 = kKvKeys * kblk + 32 * (wave >> 1);
#pragma unroll
    for (int p = 0; p < 32 * D * 2 / 1024; ++p) {
      const int pos = 64 * p + lane, row = pos / CPR, col = (pos % CPR) ^ swz<D>(row);
      buf_dma16(r, kvl + wave * TILE + 512 * p, uint32_t((int64_t(k0 + row) * rs + 8 * col) * 2));
    }
  } else {
    load_kv_operands<D>(a, b, kvh, sq, key, kf, vf);
  }
  const uint16_t* const Kw = kvl + (2 * kh) * TILE;  // this wave's K and V tiles (KVL)
  const uint16_t* const Vw = Kw + TILE;
  const float cs = a.qsign ? -a.c : a.c;  // exponent factor: scale log2(e), with its sign

  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }

  // Items: (query head h, 32-row block qb) for h < G and qb < n_qb.  Step (h, qp) stages the
  // two items (h, 2qp) and (h, 2qp + 1) -- slot 0 and slot 1 -- so a step never spans two heads.
  const int qb_lo = qlo / 32;
  const int n_qb = qhi > qlo ? (qhi + 31) / 32 - qb_lo : 0;
  const int n_qp = (n_qb + 1) / 2;
  const int n_steps = G * n_qp;

  // ---- staging.  Everything a step reads goes straight from memory into an LDS stage by DMA
  // (buffer_load ... lds): the four 32-row tiles (slot 0 Q, slot 0 dO, slot 1 Q, slot 1 dO; wave w
  // loads tile w, IPT instructions of 64 lanes x 16 bytes, each writing 1 KiB of the swizzled tile
  // in lane order -- lane l of instruction p loads the global chunk that the swizzle places at
  // 16-byte position 64p + l) and each slot's row statistics (one 64-lane dword instruction: the
  // dQ kernel stores a 32-row block's lse * log2(e) and -delta as 64 consecutive floats, exactly
  // the slot's statistics area; waves w and w + 2 both load slot w % 2's, the same bytes to the same
  // place, so that every wave issues IPT + 1 loads per step).  Loads go through buffer resources
  // spanning one query head's rows [0, L) (rows past L read as zero; a head slice is < 2^31 bytes,
  // checked by the C ABI); descriptors change only with the head.
  // NSTG stages rotate and loads are issued NSTG - 1 steps ahead, so the loads of a step have
  // NSTG - 2 steps of compute to land.
  constexpr int IPT = 32 * D * 2 / 1024;         // DMA instructions per tile (1 KiB each)
  constexpr int PER = IPT + 1;                   // loads per wave and step
  static_assert(PER <= 63, "vmcnt immediate");
  const int t_slot = wave >> 1, t_kind = wave & 1;  // this wave's tile: slot, Q (0) or dO (1)
  const int64_t t_rs = t_kind ? a.sdo[2] : a.sq[2];  // row stride of the tile's tensor
  uint32_t dma_off[IPT];
#pragma unroll
  for (int p = 0; p < IPT; ++p) {
    const int pos = 64 * p + lane;             // 16-byte position in the swizzled tile
    const int row = pos / CPR, phys = pos % CPR;
    const int col = phys ^ swz<D>(row);        // the logical chunk stored there
    dma_off[p] = uint32_t((int64_t(row) * t_rs + 8 * col) * 2);
  }
  const char* qslice = reinterpret_cast<const char*>(a.q) + 2 * slice_off(a.sq, b, kvh * G, sq.row);
  const char* dslice = reinterpret_cast<const char*>(a.dout) + 2 * slice_off(a.sdo, b, kvh * G, sq.row);
  // row statistics of (b, head kvh G + fh): Lp / 32 blocks of 64 floats
  const int nblk = a.Lp / 32;
  const char* sslice = reinterpret_cast<const char*>(a.delta + (int64_t(b) * a.Hq + int64_t(kvh) * G) * nblk * 64);
  const char* tile_slice = t_kind ? dslice : qslice;
  const int64_t t_hs = t_kind ? a.sdo[1] : a.sq[1];  // head stride of the tile's tensor
  const uint32_t nt_bytes = span_bytes(L, t_rs, D);
  const uint32_t bt = uint32_t(64 * t_rs);  // tile bytes per 32-row block
  const int s_slot = wave & 1;              // the slot whose statistics this wave loads
  // fetch side: the step (fh, fp) being loaded and the descriptors of head fh
  int fh = 0, fp = 0;
  rsrc_t rtile, rstat;
  auto set_head = [&]() {
    rtile = make_rsrc(tile_slice + int64_t(fh) * 2 * t_hs, nt_bytes);
    rstat = make_rsrc(sslice + int64_t(fh) * nblk * 256, uint32_t(nblk * 256));
  };
  // issues the loads of step (fh, fp) into LDS stage `buf` and moves the fetch side to the next
  // step (loads past the last step read the last head's rows or zeros into a stage that is never
  // computed, so every step keeps the same number of loads in flight)
  auto issue = [&](int buf) {
    const uint32_t qb0 = uint32_t(qb_lo + 2 * fp);  // block of slot 0
    const uint32_t blk_off = (qb0 + uint32_t(t_slot)) * bt;
    uint16_t* dst = lds + buf * STAGE + t_slot * SLOT + t_kind * TILE;
#pragma unroll
    for (int p = 0; p < IPT; ++p)
      buf_dma16(rtile, dst + 512 * p, dma_off[p] + blk_off);
    buf_dma4(rstat, lds + buf * STAGE + s_slot * SLOT + 2 * TILE, (qb0 + uint32_t(s_slot)) * 256u + 4u * lane);
    if (++fp == n_qp) {
      fp = 0;
      ++fh;
      if (fh < G) set_head();
    }
  };

  // Per-lane constants of the compute.  The mask is one unsigned compare per element:
  //   regular workgroup: q - k < lim, lim = W for ordinary keys, 2^31 for sink keys (any
  //     q >= k), wqhi - k for sink keys of a block whose later rows belong to chunk workgroups;
  //   chunk workgroup: q - qlo < lim, lim = qhi - qlo for sink keys, 0 for the others.
  unsigned lim;
  if (is_chunk) lim = key < S ? unsigned(qhi - qlo) : 0u;
  else lim = key < S ? (partial_block ? unsigned(max(wqhi - key, 0)) : 0x80000000u) : unsigned(W);
  const int mref = is_chunk ? qlo : key;  // mask coordinate: row - mref

  // Does this wave compute the item of block pair cp in slot hh?
  auto needed = [&](int cp) {
    const int qbi = 2 * cp + hh;
    const int qr0 = 32 * (qb_lo + qbi);
    return wave_on && qbi < n_qb && qr0 + 32 > wqlo && qr0 < wqhi && kv_half_needs(qr0, ks0, L, W, S);
  };
  // The score products of an item from LDS stage `buf`: S = Q K^T and dP - delta = dO V^T - delta
  // (the accumulator starts from -delta), lane = key column, 16 query rows per lane.
  auto scores = [&](int buf, f32x16& sacc, f32x16& dpacc) {
    const uint16_t* Qt = lds + buf * STAGE + hh * SLOT;
    const uint16_t* Dt = Qt + TILE;
    const float* ndlt = reinterpret_cast<const float*>(Qt + 2 * TILE) + 32;  // -delta
    sacc = f32x16{};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(ndlt + 8 * j + 4 * hf);
#pragma unroll
      for (int i = 0; i < 4; ++i) dpacc[4 * j + i] = d4[i];
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int a_off = swz_off<D>(r32, hf * (D / 2) + 8 * ks);
      if constexpr (KVL) {
        sacc = E::mfma(lds16(Qt + a_off), lds16(Kw + a_off), sacc);
        dpacc = E::mfma(lds16(Dt + a_off), lds16(Vw + a_off), dpacc);
      } else {
        sacc = E::mfma(lds16(Qt + a_off), kf[ks], sacc);
        dpacc = E::mfma(lds16(Dt + a_off), vf[ks], dpacc);
      }
    }
  };
  // The rest of an item, from its score products and LDS stage `buf`: P = exp2(s c - lse2) and
  // dS = P (dP - delta) elementwise (masked or not), then dV^T += dO^T P and dK^T += Q^T dS with P
  // and dS straight from registers and dO^T / Q^T read transposed from the row-major tiles.
  auto finish = [&](int buf, int cp, const f32x16& sacc, const f32x16& dpacc) {
    const int qr0 = 32 * (qb_lo + 2 * cp + hh);
    const uint16_t* Qt = lds + buf * STAGE + hh * SLOT;
    const float* lse2 = reinterpret_cast<const float*>(Qt + 2 * TILE);
    const bool full = !is_chunk && qr0 >= wqlo && qr0 + 32 <= wqhi && tile_full(ks0, qr0, W, S);
    const int m0 = qr0 + 4 * hf - mref;  // mask coordinate of register e = 0
    float p[16], ds[16];
    auto elementwise = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse2 + 8 * j + 4 * hf);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * j + i;
          float pe = fast_exp2(fmaf(sacc[e], cs, -l4[i]));
          if constexpr (MASK) pe = unsigned(m0 + 8 * j + i) < lim ? pe : 0.f;
          p[e] = pe;
          ds[e] = pe * dpacc[e];
        }
      }
    };
    // D = 64: the rest of the item at a higher issue priority than the score products of the other
    // workgroup's wave on the SIMD (as the forward's softmax): c3 1217 -> 1164 us, c2 34.5 -> 33.8
    // us; D = 16 and 128 measured no gain
    if constexpr (D == 64) __builtin_amdgcn_s_setprio(1);
    // D = 128 (one wave per SIMD): the mask is applied to every item (it keeps every element of a
    // full one), so that the score products, the elementwise work and the dV/dK products form one
    // basic block that the scheduler can interleave (c5 dK/dV 361 -> 355 us)
    if (D != 128 && full) elementwise(std::false_type{});
    else elementwise(std::true_type{});
    const u32x4 pb[2] = {pack8<E>(p), pack8<E>(p + 8)};
    const u32x4 sb[2] = {pack8<E>(ds), pack8<E>(ds + 8)};
    dkdv_products<E, D, DB>(Qt, Qt + TILE, pb, sb, dv, dk);
    if constexpr (D == 64) __builtin_amdgcn_s_setprio(0);
  };

  // Descriptors are built before any load, whatever the number of steps (a workgroup can own
  // no items: a chunk whose rows all lie inside the window).
  set_head();
  // Stage s % NSTG holds step s; the loads of step s + NSTG - 1 go into stage (s - 1) % NSTG, whose
  // last reader (step s - 1) is behind the barrier at the start of step s; the wait before that
  // barrier is for this wave's own loads of step s (the explicit wait: the compiler does not track
  // the DMA writes into LDS and would otherwise wait for every load in flight).
  if (n_steps > 0) {
    // loads NSTG - 1 steps ahead; step s waits for its own
    for (int k = 0; k < NSTG - 1; ++k) issue(k);
    if constexpr (!KVL) kv_operands_ready(kf, vf);
    int cp = 0, cur = 0, nxt = NSTG - 1;  // stage of step s, stage of step s + NSTG - 1
    for (int s = 0; s < n_steps; ++s) {
      wait_vm_lgkm0_barrier<(NSTG - 2) * PER>();  // step s landed everywhere
      // (D = 128 issues after its compute: measured 4% faster there, slower at D = 64)
      if constexpr (D != 128) issue(nxt);
      if (needed(cp)) {
        f32x16 sacc, dpacc;
        scores(cur, sacc, dpacc);
        finish(cur, cp, sacc, dpacc);
      }
      if constexpr (D == 128) issue(nxt);
      cp = cp + 1 == n_qp ? 0 : cp + 1;
      cur = cur + 1 == NSTG ? 0 : cur + 1;
      nxt = nxt + 1 == NSTG ? 0 : nxt + 1;
    }
  }

  // ---- add the two head slots' partial sums (hh = 0 gets hh = 1's), fixed order ---------------
  // The stages are reused: nothing may still be landing in them.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
  if (hh == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        red[((kh * 2 + 0) * DB * 16 + db * 16 + e) * 64 + lane] = dk[db][e];
        red[((kh * 2 + 1) * DB * 16 + db * 16 + e) * 64 + lane] = dv[db][e];
      }
  }
  __syncthreads();
  if (hh == 0) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        dk[db][e] += red[((kh * 2 + 0) * DB * 16 + db * 16 + e) * 64 + lane];
        dv[db][e] += red[((kh * 2 + 1) * DB * 16 + db * 16 + e) * 64 + lane];
      }
  }

  // ---- outputs: lane (key, hf) holds head-dim indices 32db + 16hf + e (D == 16: hf == 0) ------
  float* pk = nullptr;
  if (partial_block) {
    const int64_t blk = (int64_t(b) * a.Hkv + kvh) * a.nsp + kblk;
    const int slot = is_chunk ? chunk : a.n_chunks;
    pk = a.partial + (blk * (a.n_chunks + 1) + slot) * 2 * a.srows * D;
  }
  if (hh == 0 && key < L) {
    const bool sink_row = partial_block && key < S;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      if (D == 16 && hf == 1) continue;
      const int d0 = 32 * db + (D >= 32 ? 16 * hf : 0);
      if (sink_row) {
        float* rk = pk + (32 * kh + r32) * D + d0;  // row key - 64 kblk < srows
        float* rv = rk + a.srows * D;
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          *reinterpret_cast<f32x4*>(rk + 4 * e4) =
              f32x4{dk[db][4 * e4], dk[db][4 * e4 + 1], dk[db][4 * e4 + 2], dk[db][4 * e4 + 3]};
          *reinterpret_cast<f32x4*>(rv + 4 * e4) =
              f32x4{dv[db][4 * e4], dv[db][4 * e4 + 1], dv[db][4 * e4 + 2], dv[db][4 * e4 + 3]};
        }
      } else if (!is_chunk) {
        char* dkp = reinterpret_cast<char*>(a.dk) + 2 * slice_off(a.sdk, b, kvh, sq.row + key);
        char* dvp = reinterpret_cast<char*>(a.dv) + 2 * slice_off(a.sdv, b, kvh, sq.row + key);
        float kv[16], vv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          kv[e] = dk[db][e] * a.scale;
          vv[e] = dv[db][e];
        }
        st16(dkp + 2 * d0, pack8<E>(kv));
        st16(dkp + 2 * (d0 + 8), pack8<E>(kv + 8));
        st16(dvp + 2 * d0, pack8<E>(vv));
        st16(dvp + 2 * (d0 + 8), pack8<E>(vv + 8));
      }
    }
  }

  // dq_sink_mode with at most 256 (sink key, column) pairs: key block 0's workgroup folds its
  // sink keys (see fold_sink_keys); the barrier makes its own slot writes visible to all its
  // threads, and every thread is past its last read of the LDS that the fold reuses.
  if (partial_block && !is_chunk && dkdv_folds_in_kernel(a, D, KVL)) {
    __syncthreads();
    fold_sink_keys<E, D>(b, kvh, min(min(S, kKvKeys), L), sq, reinterpret_cast<float*>(lds));
  }
}

// ---------------------------------------------------------------------------------------------
// dK / dV with 32-key workgroups (bwd_dkdv4_kernel), for window shapes without chunked sink rows
// and KV groups of a multiple of 4 query heads (launch_bwd_dkdv picks it; dkdv4_eligible).  A
// workgroup owns the 32 keys [ks0, ks0 + 32) of one KV head; its NW waves (4, or 8 / 16 for large
// KV groups on small grids, dkdv4_waves) all hold those keys' K^T / V^T fragments and dK/dV
// accumulators, and each takes one query head of every group of NW: step (g, qb) is head
// NW g + wave, 32-row block qb.  Every wave therefore needs the same row blocks, so no wave idles on
// a block only the other key half sees (bwd_dkdv_kernel's 2-tile steps leave a quarter of its
// wave-steps idle at W = 128), and the rows of a 32-key half are fewer than those of a 64-key
// block.  Each wave stages its own items -- its Q and dO tiles and row statistics -- by DMA into its
// own slot of a 2-stage LDS ring, one step ahead, and waits only for its own loads: the step loop
// has no barrier.  At the end the waves' sums are added in LDS in a fixed order (in wave order for
// 4 waves, pairwise in rounds for more).
// The per-item mathematics is bwd_dkdv_kernel's.
// ---------------------------------------------------------------------------------------------
template <int D, int NW = 4>
__host__ __device__ constexpr int dkdv4_lds_elems() {
  const int stages = 2 * NW * (2 * 32 * D + 128);
  // fp32 partials of the waves that hand theirs on in the first round of the wave sum (NW / 2
  // of them; NW = 4: waves 1..3 in one round)
  const int red = (NW == 4 ? 3 : NW / 2) * 2 * (D >= 32 ? D / 32 : 1) * 16 * 64 * 2;
  return stages > red ? stages : red;
}

// Does key block 0's workgroup of bwd_dkdv4_kernel fold the sink keys itself (as
// dkdv_folds_in_kernel for bwd_dkdv_kernel, with this kernel's LDS)?
__host__ __device__ inline bool dkdv4_folds_in_kernel(const Args& a, int D, int lds_elems) {
  return a.sink_dq && (a.S < kKvKeys ? a.S : kKvKeys) * D <= 256 &&
         ((a.dq_wgs + 3) & ~3) + 4 * 256 <= lds_elems / 2;
}

template <typename E, int D, int NW = 4>
__global__ __launch_bounds__(64 * NW, NW == 16 ? 4 : D == 16 && NW == 4 ? 3 : 2) void bwd_dkdv4_kernel(const Args a) {
  constexpr int KS = D / 16;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int TILE = 32 * D;
  constexpr int SLOT = 2 * TILE + 128;  // Q, dO, then lse2[32] and -delta[32] as fp32
  constexpr int STAGE = NW * SLOT;      // one slot per wave
  constexpr int CPR = D / 8;
  constexpr int IPT = 32 * D * 2 / 1024;  // DMA instructions per tile (1 KiB each)
  constexpr int PER = 2 * IPT + 1;        // loads per wave and step
  static_assert(PER <= 63, "vmcnt immediate");
  constexpr int LDS_ELEMS = dkdv4_lds_elems<D, NW>();
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hf = lane >> 5;
  const int W = a.W, S = a.S, G = a.G;

  // workgroups grouped per (b, KV head), n_kblocks 32-key blocks each, groups in (KV head, batch)
  // order with the KV head outermost (as bwd_dkdv_kernel)
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int grp = id / a.n_kblocks, kblk = id % a.n_kblocks;
  const int kvh = grp / a.B, b = grp % a.B;
  const Seq sq = seq_of(a, b);
  const int L = sq.L;
  const int ks0 = 32 * kblk;
  if (ks0 >= L) return;
  const bool partial_block = a.sink_dq && kblk == 0;  // its sink keys' rows continue in the dQ kernel
  const int key = ks0 + r32;
  const int qlo = ks0, qhi = kv4_rows_end(ks0, L, W, S, a.sink_dq != 0);

  u32x4 kf[KS], vf[KS];
  load_kv_operands<D>(a, b, kvh, sq, key, kf, vf);
  const float cs = a.qsign ? -a.c : a.c;  // exponent factor: scale log2(e), with its sign
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }

  // steps: (head group g, row block qb), g outermost so that descriptors change once per group
  const int qb_lo = qlo / 32;
  const int n_qb = qhi > qlo ? (qhi + 31) / 32 - qb_lo : 0;
  const int n_steps = (G / NW) * n_qb;

  // staging: this wave's Q and dO tiles (IPT instructions each, lane l of instruction p loading the
  // global chunk that the swizzle places at 16-byte position 64p + l) and its row statistics
  // (instruction p covers rows 64p / CPR + lane / CPR: the same swizzle for every p, as the swizzle
  // depends on the row mod 8 only and 64 / CPR is a multiple of 8)
  static_assert((64 / CPR) % 8 == 0, "row step of one DMA instruction");
  const int row0 = lane / CPR, col0 = (lane % CPR) ^ swz<D>(row0);
  const uint32_t q_off0 = uint32_t((int64_t(row0) * a.sq[2] + 8 * col0) * 2);
  const uint32_t d_off0 = uint32_t((int64_t(row0) * a.sdo[2] + 8 * col0) * 2);
  const uint32_t q_step = uint32_t((64 / CPR) * a.sq[2] * 2), d_step = uint32_t((64 / CPR) * a.sdo[2] * 2);
  const uint32_t bq = uint32_t(64 * a.sq[2]), bd = uint32_t(64 * a.sdo[2]);  // bytes per 32-row block
  const int nblk = a.Lp / 32;
  const uint32_t q_bytes = span_bytes(L, a.sq[2], D), d_bytes = span_bytes(L, a.sdo[2], D);
  int fg = -1;  // head group of the current descriptors
  rsrc_t rq, rd, rs;
  auto issue = [&](int s, int buf) {
    const int g = s / n_qb, qb = qb_lo + s % n_qb;
    if (g != fg) {
      fg = g;
      const int h = kvh * G + NW * g + wave;
      rq = make_rsrc(reinterpret_cast<const char*>(a.q) + 2 * slice_off(a.sq, b, h, sq.row), q_bytes);
      rd = make_rsrc(reinterpret_cast<const char*>(a.dout) + 2 * slice_off(a.sdo, b, h, sq.row), d_bytes);
      rs = make_rsrc(reinterpret_cast<const char*>(a.delta + (int64_t(b) * a.Hq + h) * nblk * 64), uint32_t(nblk * 256));
    }
    uint16_t* dst = lds + buf * STAGE + wave * SLOT;
#pragma unroll
    for (int p = 0; p < IPT; ++p) {
      buf_dma16(rq, dst + 512 * p, q_off0 + uint32_t(p) * q_step + uint32_t(qb) * bq);
      buf_dma16(rd, dst + TILE + 512 * p, d_off0 + uint32_t(p) * d_step + uint32_t(qb) * bd);
    }
    buf_dma4(rs, dst + 2 * TILE, uint32_t(qb) * 256u + 4u * lane);
  };

  unsigned lim;
  lim = key < S ? (partial_block ? unsigned(max(qhi - key, 0)) : 0x80000000u) : unsigned(W);
  // The item of step s: S = Q K^T and dP - delta (accumulated from -delta), then P and dS
  // elementwise and dV^T += dO^T P, dK^T += Q^T dS (bwd_dkdv_kernel's scores / finish).
  auto item = [&](int buf, int qb) {
    const uint16_t* Qt = lds + buf * STAGE + wave * SLOT;
    const uint16_t* Dt = Qt + TILE;
    const float* lse2 = reinterpret_cast<const float*>(Qt + 2 * TILE);
    const float* ndlt = lse2 + 32;
    const int qr0 = 32 * qb;
    f32x16 sacc = f32x16{}, dpacc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(ndlt + 8 * j + 4 * hf);
#pragma unroll
      for (int i = 0; i < 4; ++i) dpacc[4 * j + i] = d4[i];
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int a_off = swz_off<D>(r32, hf * (D / 2) + 8 * ks);
      sacc = E::mfma(lds16(Qt + a_off), kf[ks], sacc);
      dpacc = E::mfma(lds16(Dt + a_off), vf[ks], dpacc);
    }
    const bool full = qr0 + 32 <= qhi && tile_full(ks0, qr0, W, S);
    const int m0 = qr0 + 4 * hf - key;
    float p[16], ds[16];
    auto elementwise = [&](auto mask_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse2 + 8 * j + 4 * hf);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * j + i;
          float pe = fast_exp2(fmaf(sacc[e], cs, -l4[i]));
          if constexpr (MASK) pe = unsigned(m0 + 8 * j + i) < lim ? pe : 0.f;
          p[e] = pe;
          ds[e] = pe * dpacc[e];
        }
      }
    };
    if (full) elementwise(std::false_type{});
    else elementwise(std::true_type{});
    const u32x4 pb[2] = {pack8<E>(p), pack8<E>(p + 8)};
    const u32x4 sb[2] = {pack8<E>(ds), pack8<E>(ds + 8)};
    dkdv_products<E, D, DB>(Qt, Qt + TILE, pb, sb, dv, dk);
  };

  if (n_steps > 0) {
    issue(0, 0);
    kv_operands_ready(kf, vf);
    for (int s = 0; s < n_steps; ++s) {
      // the next step's items into the other stage (its last reader is this wave's previous
      // step), then wait for this step's
      if (s + 1 < n_steps) {
        issue(s + 1, (s + 1) & 1);
        wait_vm_lgkm0<PER>();
      } else {
        wait_vm_lgkm0<0>();
      }
      const int qb = qb_lo + s % n_qb;
      if (kv_half_needs(32 * qb, ks0, L, W, S)) item(s & 1, qb);  // (the same on every wave)
    }
  }

  // ---- add the waves' sums into wave 0, in a fixed order: with 4 waves, waves 1..3's in wave
  // order; with more, pairwise in rounds (round r: wave w with w % 2r == r hands its sum to w - r)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
  constexpr int RW = 2 * DB * 16 * 64;  // floats of one wave's sums
  auto put = [&](int region) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        red[region * RW + ((0 * DB + db) * 16 + e) * 64 + lane] = dk[db][e];
        red[region * RW + ((1 * DB + db) * 16 + e) * 64 + lane] = dv[db][e];
      }
  };
  auto add = [&](int region) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        dk[db][e] += red[region * RW + ((0 * DB + db) * 16 + e) * 64 + lane];
        dv[db][e] += red[region * RW + ((1 * DB + db) * 16 + e) * 64 + lane];
      }
  };
  if constexpr (NW == 4) {
    if (wave > 0) put(wave - 1);
    __syncthreads();
    if (wave == 0) {
#pragma unroll 1  // (one wave's sums at a time: unrolled, all 3 * 32 * DB loads are live at once)
      for (int w = 0; w < 3; ++w) add(w);
    }
  } else {
#pragma unroll 1
    for (int r = 1; r < NW; r *= 2) {
      if (wave % (2 * r) == r) put(wave / (2 * r));
      __syncthreads();
      if (wave % (2 * r) == 0) add(wave / (2 * r));
      __syncthreads();  // (the regions are written again in the next round)
    }
  }

  // ---- outputs: lane (key, hf) holds head-dim indices 32db + 16hf + e (D == 16: hf == 0) ------
  if (wave == 0 && key < L) {
    const bool sink_row = partial_block && key < S;
    // key block 0's slot of the sink partials (the layout of bwd_dkdv_kernel's)
    const int64_t blk = int64_t(b * a.Hkv + kvh) * a.nsp;
    float* pk = partial_block ? a.partial + (blk * (a.n_chunks + 1) + a.n_chunks) * 2 * a.srows * D : nullptr;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      if (D == 16 && hf == 1) continue;
      const int d0 = 32 * db + (D >= 32 ? 16 * hf : 0);
      if (sink_row) {
        float* rk = pk + r32 * D + d0;  // key < srows
        float* rv = rk + a.srows * D;
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          *reinterpret_cast<f32x4*>(rk + 4 * e4) =
              f32x4{dk[db][4 * e4], dk[db][4 * e4 + 1], dk[db][4 * e4 + 2], dk[db][4 * e4 + 3]};
          *reinterpret_cast<f32x4*>(rv + 4 * e4) =
              f32x4{dv[db][4 * e4], dv[db][4 * e4 + 1], dv[db][4 * e4 + 2], dv[db][4 * e4 + 3]};
        }
      } else {
        char* dkp = reinterpret_cast<char*>(a.dk) + 2 * slice_off(a.sdk, b, kvh, sq.row + key);
        char* dvp = reinterpret_cast<char*>(a.dv) + 2 * slice_off(a.sdv, b, kvh, sq.row + key);
        float kv[16], vv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          kv[e] = dk[db][e] * a.scale;
          vv[e] = dv[db][e];
        }
        st16(dkp + 2 * d0, pack8<E>(kv));
        st16(dkp + 2 * (d0 + 8), pack8<E>(kv + 8));
        st16(dvp + 2 * d0, pack8<E>(vv));
        st16(dvp + 2 * (d0 + 8), pack8<E>(vv + 8));
      }
    }
  }
  if (partial_block && dkdv4_folds_in_kernel(a, D, LDS_ELEMS)) {
    __syncthreads();
    fold_sink_keys<E, D>(b, kvh, min(min(S, kKvKeys), L), sq, reinterpret_cast<float*>(lds));
  }
}

// ---------------------------------------------------------------------------------------------
// Sink fold: the dK/dV rows of the split sink keys are the sum of fp32 partials: those the
// dK/dV kernel's regular and chunk workgroups wrote for them and, in dq_sink_mode, those the dQ
// kernel flushed (the flagged tiles of the (batch, KV head)).
// fold_sink_key adds them for one sink key with the 256 threads of a workgroup: thread (g, d)
// adds slots g, g + NG, g + 2 NG, ... (their loads in flight together), then the NG group sums
// are added in order g = 0, 1, ... -- a fixed order, so results are deterministic.
// bwd_sink_fold_kernel runs it in a launch of its own after the dK/dV kernel (every partial is
// then visible without a device-wide fence).  In dq_sink_mode the dQ kernel's slots are complete
// before the dK/dV kernel starts and the only other partial is that of key block 0's own
// workgroup, so when the sink keys' (key, column) pairs fit one pass of 256 threads that
// workgroup folds them itself after writing its slot (fold_sink_keys) and no fold launch follows.
// ---------------------------------------------------------------------------------------------
template <typename E, int D>
__device__ void fold_sink_key(int b, int kvh, int key, const Seq& sq, float (&part)[2][256 / D][D]) {
  KArgs& Ak = args_fresh();
  constexpr int NG = 256 / D;  // slot groups
  constexpr int kBatch = 16;
  const int bh = b * Ak.Hkv + kvh;
  const int kblk = key / kKvKeys, row = key % kKvKeys;
  const int d = threadIdx.x % D, g = threadIdx.x / D;
  const int64_t blk = int64_t(bh) * Ak.nsp + kblk;
  const int64_t slot_stride = int64_t(2) * Ak.srows * D;
  const float* src = Ak.partial + blk * (Ak.n_chunks + 1) * slot_stride + row * D + d;
  const int ns = Ak.n_chunks + 1;
  float sk = 0.f, sv = 0.f;
  for (int s0 = g; s0 < ns; s0 += NG * kBatch) {
    float xk[kBatch], xv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int sl = s0 + j * NG;
      const bool in = sl < ns;
      const float* p = src + int64_t(in ? sl : 0) * slot_stride;
      xk[j] = in ? p[0] : 0.f;
      xv[j] = in ? p[Ak.srows * D] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      sk += xk[j];
      sv += xv[j];
    }
  }
  if (Ak.sink_dq && Ak.dq_slide) {
    // the sliding dQ kernel's units of (b, KV head) that own tiles, in (head group, chunk) order
    const int hgn = Ak.G / 8, ncu = Ak.slide_ncu;
    const int nv = min(ncu, ((sq.L + 31) / 32 + Ak.slide_ct - 1) / Ak.slide_ct);
    const int base = (kvh * Ak.B + b) * hgn * ncu, n = hgn * nv;
    const int n_out = 2 * Ak.srows * D;
    const float* dsrc = Ak.dq_sink_part + row * D + d;
    for (int j0 = g; j0 < n; j0 += NG * kBatch) {
      float xk[kBatch], xv[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int jj = j0 + j * NG, i = jj < n ? jj : 0;
        const float* p = dsrc + int64_t(base + (i / nv) * ncu + i % nv) * n_out;
        xk[j] = jj < n ? p[0] : 0.f;
        xv[j] = jj < n ? p[Ak.srows * D] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        sk += xk[j];
        sv += xv[j];
      }
    }
  } else if (Ak.sink_dq) {
    // The dQ kernel's flushed partials of this (b, KV head) = tiles [(b + B kvh) tpk, + tpk): on
    // XCD x, whose tiles are [x_lo, x_hi) and whose Ak.dq_wgs / 8 workgroups stride through them,
    // the runs start at the first Ak.dq_wgs / 8 tiles of [max(x_lo, lo), min(x_hi, hi)).  All the
    // loads are independent; slots are added in (XCD, tile) order.
    constexpr int nx = 8;
    const int tpk = Ak.n_qtiles * (Ak.G / Ak.wh);
    const int n_tiles = tpk * Ak.B * Ak.Hkv;
    const int wgs_x = Ak.dq_wgs / nx;
    const int lo = (b + Ak.B * kvh) * tpk, hi = lo + tpk;
    const int per = n_tiles / nx, rem = n_tiles % nx;
    const int n_out = 2 * Ak.srows * D;
    const float* dsrc = Ak.dq_sink_part + row * D + d;
    for (int x = 0; x < nx; ++x) {
      const int x_lo = x * per + min(x, rem), x_hi = x_lo + per + (x < rem ? 1 : 0);
      const int A = max(x_lo, lo), B = min(x_hi, hi);
      const int n = B > A ? min(wgs_x, B - A) : 0;
      for (int j0 = g; j0 < n; j0 += NG * kBatch) {
        float xk[kBatch], xv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int jj = j0 + j * NG;
          const float* p = dsrc + int64_t(A + (jj < n ? jj : 0)) * n_out;
          xk[j] = jj < n ? p[0] : 0.f;
          xv[j] = jj < n ? p[Ak.srows * D] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          sk += xk[j];
          sv += xv[j];
        }
      }
    }
  }
  part[0][g][d] = sk;
  part[1][g][d] = sv;
  __syncthreads();
  if (g == 0) {
    float tk = 0.f, tv = 0.f;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      tk += part[0][j][d];
      tv += part[1][j][d];
    }
    const uint32_t pk = E::pack2(tk * Ak.scale, tv);
    reinterpret_cast<uint16_t*>(Ak.dk)[slice_off(Ak.sdk, b, kvh, sq.row + key) + d] = uint16_t(pk);
    reinterpret_cast<uint16_t*>(Ak.dv)[slice_off(Ak.sdv, b, kvh, sq.row + key) + d] = uint16_t(pk >> 16);
  }
  __syncthreads();  // part is free again
}

// fold_sink_keys: the same sums for all nk sink keys at once, in key block 0's workgroup.  A slot's
// 2 nk D values (dK rows, then dV rows) are C = nk D / 2 chunks of four floats; thread t < P C
// (P = 256 / C slot groups) takes chunk t % C of the slots at positions j, j + P, j + 2P, ...
// (j = t / C) of the list [own slot, the dQ kernel's run slots in (XCD, tile) order], kBatch
// 16-byte loads in flight at a time; the P group sums of a chunk are then added in LDS in order
// j = 0, 1, ....  With C > 256 (D = 128 and up to 16 sink keys) thread t takes the chunks t,
// t + 256, ... over the whole list.  `smem` is the kernel's LDS, free at this point (dq_wgs run
// indices, then the P C chunk sums).
template <typename E, int D>
__device__ void fold_sink_keys(int b, int kvh, int nk, const Seq& sq, float* smem) {
  KArgs& Ak = args_fresh();
  constexpr int kBatch = D <= 32 ? 8 : 32;  // 4 kBatch registers per thread (D <= 32: <= 128 in all)
  const int t = threadIdx.x;
  const int Q = nk * D / 4;  // chunks per half
  const int C = 2 * Q;
  const int P = 256 / C;
  const int srd = Ak.srows * D;  // floats of a half slot
  const int64_t slot_stride = int64_t(2) * srd;
  // the run slots of this (b, KV head): on XCD x, whose tiles are [x_lo, x_hi) and whose
  // Ak.dq_wgs / 8 workgroups stride through them, the runs start at the first Ak.dq_wgs / 8 tiles
  // of [max(x_lo, lo), min(x_hi, hi)) (see the dQ kernel's flush)
  int* runs = reinterpret_cast<int*>(smem);
  float* red = smem + ((Ak.dq_wgs + 3) & ~3);
  int nr = 0;
  if (Ak.dq_slide) {
    // the sliding dQ kernel's units of (b, KV head) that own tiles, in (head group, chunk) order
    const int hgn = Ak.G / 8, ncu = Ak.slide_ncu;
    const int nv = min(ncu, ((sq.L + 31) / 32 + Ak.slide_ct - 1) / Ak.slide_ct);
    const int base = (kvh * Ak.B + b) * hgn * ncu;
    nr = hgn * nv;
    for (int i = t; i < nr && t < 256; i += 256) runs[i] = base + (i / nv) * ncu + i % nv;
  } else {
    constexpr int nx = 8;
    const int tpk = Ak.n_qtiles * (Ak.G / Ak.wh);
    const int n_tiles = tpk * Ak.B * Ak.Hkv;
    const int wgs_x = Ak.dq_wgs / nx;
    const int lo = (b + Ak.B * kvh) * tpk, hi = lo + tpk;
    const int per = n_tiles / nx, rem = n_tiles % nx;
    for (int x = 0; x < nx; ++x) {
      const int x_lo = x * per + min(x, rem), x_hi = x_lo + per + (x < rem ? 1 : 0);
      const int r_lo = max(x_lo, lo), r_hi = min(x_hi, hi);
      const int n = r_hi > r_lo ? min(wgs_x, r_hi - r_lo) : 0;
      for (int i = t; i < n && t < 256; i += 256) runs[nr + i] = r_lo + i;
      nr += n;
    }
  }
  __syncthreads();
  // chunk c of the output (c < Q: dK, else dV): total tot, scaled and stored as 16-bit
  auto store_chunk = [&](int cc, const f32x4& tot) {
    const bool is_dk = cc < Q;
    const int e = 4 * (is_dk ? cc : cc - Q), key = e / D, col = e % D;
    const float m = is_dk ? Ak.scale : 1.f;
    const u32x2 out = {E::pack2(tot[0] * m, tot[1] * m), E::pack2(tot[2] * m, tot[3] * m)};
    char* base = reinterpret_cast<char*>(is_dk ? Ak.dk : Ak.dv);
    const int64_t at = is_dk ? slice_off(Ak.sdk, b, kvh, sq.row + key) : slice_off(Ak.sdv, b, kvh, sq.row + key);
    *reinterpret_cast<u32x2*>(base + 2 * (at + col)) = out;
  };
  if (C > 256) {
    // more chunks than threads: each thread sums whole chunks, the workgroup's own slot first and
    // then the runs in order
    const int64_t blk = int64_t(b * Ak.Hkv + kvh) * Ak.nsp;
    const float* own = Ak.partial + blk * (Ak.n_chunks + 1) * slot_stride;
    for (int cc = t; cc < C; cc += 256) {
      const int off = cc < Q ? 4 * cc : srd + 4 * (cc - Q);
      f32x4 tot = *reinterpret_cast<const f32x4*>(own + off);
      const float* dsrc = Ak.dq_sink_part + off;
      for (int i0 = 0; i0 < nr; i0 += kBatch) {
        f32x4 x[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int i = i0 + u;
          x[u] = *reinterpret_cast<const f32x4*>(dsrc + int64_t(runs[i < nr ? i : 0]) * slot_stride);
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          if (i0 + u < nr) {
            tot[0] += x[u][0];
            tot[1] += x[u][1];
            tot[2] += x[u][2];
            tot[3] += x[u][3];
          }
        }
      }
      store_chunk(cc, tot);
    }
    return;
  }
  const int c = t % C, j = t / C;
  const int off = c < Q ? 4 * c : srd + 4 * (c - Q);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (j < P) {
    if (j == 0) {  // the workgroup's own slot (key block 0) comes first
      const int64_t blk = int64_t(b * Ak.Hkv + kvh) * Ak.nsp;
      acc = *reinterpret_cast<const f32x4*>(Ak.partial + blk * (Ak.n_chunks + 1) * slot_stride + off);
    }
    const float* dsrc = Ak.dq_sink_part + off;
    for (int i0 = j; i0 < nr; i0 += P * kBatch) {
      f32x4 x[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = i0 + u * P;
        x[u] = *reinterpret_cast<const f32x4*>(dsrc + int64_t(runs[i < nr ? i : 0]) * slot_stride);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (i0 + u * P < nr) {
          acc[0] += x[u][0];
          acc[1] += x[u][1];
          acc[2] += x[u][2];
          acc[3] += x[u][3];
        }
      }
    }
    *reinterpret_cast<f32x4*>(red + 4 * (j * C + c)) = acc;
  }
  __syncthreads();
  if (t < C) {
    f32x4 tot = *reinterpret_cast<const f32x4*>(red + 4 * t);
    for (int g = 1; g < P; ++g) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(red + 4 * (g * C + t));
      tot[0] += v[0];
      tot[1] += v[1];
      tot[2] += v[2];
      tot[3] += v[3];
    }
    store_chunk(t, tot);
  }
}

template <typename E, int D>
__global__ __launch_bounds__(256) void bwd_sink_fold_kernel(const Args a) {
  __shared__ float part[2][256 / D][D];
  const int nrows = min(a.S, kKvKeys * a.nsp);  // sink keys of the chunked blocks
  const int key = blockIdx.x % nrows;
  const int bh = blockIdx.x / nrows;  // b * Hkv + kvh
  const int kvh = bh % a.Hkv, b = bh / a.Hkv;
  const Seq sq = seq_of(a, b);
  if (key >= sq.L) return;  // a sink key past the end of a short sequence: no such row
  fold_sink_key<E, D>(b, kvh, key, sq, part);
}

// The D = 128 dQ and dK/dV kernels and the D = 64 dQ kernel without sink rows are instantiated in
// fa_bwd_wide.hip, which includes this file
// with FA_BWD_WIDE_TU defined and is compiled with another machine scheduler; everything below
// belongs to this translation unit only.
#ifndef FA_BWD_WIDE_TU
extern template __global__ void bwd_dq_kernel<BF16, 64, false>(const Args);
extern template __global__ void bwd_dq_kernel<F16, 64, false>(const Args);
extern template __global__ void bwd_dq_kernel<BF16, 128, false>(const Args);
extern template __global__ void bwd_dq_kernel<BF16, 128, true>(const Args);
extern template __global__ void bwd_dq_kernel<F16, 128, false>(const Args);
extern template __global__ void bwd_dq_kernel<F16, 128, true>(const Args);
extern template __global__ void bwd_dkdv_kernel<BF16, 128>(const Args);
extern template __global__ void bwd_dkdv_kernel<F16, 128>(const Args);

// ---------------------------------------------------------------------------------------------
// Gradient of the learned sink logits: dsink[h] = sum over (b, 32-row block) of the dQ kernel's
// partials, in a fixed order (each thread strides over the partials in order, then the waves'
// sums are combined in wave order), so reruns are bitwise identical.  One workgroup per head.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void bwd_sink_logit_kernel(const Args a) {
  __shared__ float wsum[4];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int nb = a.Lp / 32;
  const int64_t n = int64_t(a.B) * nb;
  float acc = 0.f;
  for (int64_t i = tid; i < n; i += 256) {
    const int64_t b = i / nb, j = i % nb;
    // row blocks past the end of a short sequence hold no partial
    if (32 * j < seq_of(a, int(b)).L) acc += a.dsink_part[(b * a.Hq + h) * nb + j];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  if ((tid & 63) == 0) wsum[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) a.dsink[h] = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
}

// ---------------------------------------------------------------------------------------------
// Packed rows outside every sequence (see TailArgs): one thread per (row, head) of each tensor, in
// a grid-stride loop over the uncovered rows.  With cu_seqlens[0] = 0 and cu_seqlens[B] =
// total_rows (the usual case) every workgroup reads two offsets and exits.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void varlen_tail_kernel(const TailArgs t) {
  const int total = t.total_rows;
  int lo = t.cu_seqlens[0], hi = t.cu_seqlens[t.batch];
  lo = lo < 0 ? 0 : (lo > total ? total : lo);
  hi = hi < lo ? lo : (hi > total ? total : hi);
  const int64_t n_rows = int64_t(lo) + (total - hi);  // uncovered rows, [0, lo) then [hi, total)
  if (n_rows == 0) return;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int i = 0; i < t.n; ++i) {
    const int64_t units = n_rows * t.heads[i];
    for (int64_t u = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; u < units; u += stride) {
      const int64_t r = u / t.heads[i];
      const int h = int(u % t.heads[i]);
      const int64_t row = r < lo ? r : hi + (r - lo);
      char* p = static_cast<char*>(t.ptr[i]) + (h * t.head_stride[i] + row * t.row_stride[i]) * t.elem_bytes[i];
      if (t.elem_bytes[i] == 4) {
        for (int c = 0; c < t.cols[i]; ++c) reinterpret_cast<uint32_t*>(p)[c] = t.fill[i];
      } else {
        const uint32_t f2 = (t.fill[i] & 0xffffu) * 0x10001u;
        for (int c = 0; c < t.cols[i]; c += 8) st16(p + 2 * c, u32x4{f2, f2, f2, f2});  // rows 16-byte aligned
      }
    }
  }
}

hipError_t launch_varlen_tail(const TailArgs& t, hipStream_t stream) {
  hipLaunchKernelGGL(varlen_tail_kernel, dim3(256), dim3(256), 0, stream, t);
  return hipGetLastError();
}

// Resident workgroups per CU of a kernel (hipOccupancyMaxActiveBlocksPerMultiprocessor,
// 256 threads), remembered per kernel (one cache per template argument, i.e. per kernel): it
// depends only on the kernel's resources.
template <auto Kernel>
static int resident_per_cu() {
  static int cached = 0;  // benign race: every thread computes the same value
  if (cached == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, Kernel, 256, 0) != hipSuccess || n < 1) n = 1;
    cached = n;
  }
  return cached;
}

static int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n < 1)
    n = 256;
  return n;
}

// Grid of the dQ kernel: one resident wave of workgroups, a multiple of the 8 XCDs (the sink
// fold recomputes it to find the dQ kernel's sink slots).
template <typename E, int D, bool SINK>
static int dq_grid(const Args& a) {
  const int n_tiles = a.n_qtiles * (a.B * a.Hq / a.wh);
  const int slots = resident_per_cu<bwd_dq_kernel<E, D, SINK>>() * device_cus();
  return 8 * ((min(n_tiles, slots) + 7) / 8);
}

template <typename E, int D, bool SINK>
static hipError_t launch_dq_s(const Args& a, hipStream_t stream) {
  hipLaunchKernelGGL((bwd_dq_kernel<E, D, SINK>), dim3(dq_grid<E, D, SINK>(a)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <typename E, int D>
static hipError_t launch_dq_d(const Args& a, int, hipStream_t stream) {
  return a.sink_dq ? launch_dq_s<E, D, true>(a, stream) : launch_dq_s<E, D, false>(a, stream);
}

// bwd_dkdv4_kernel serves 16-bit D <= 64 with KV groups of a multiple of 4 query heads, windows of
// 1..512 keys and no chunked sink rows (no sink keys past their block's window, or dq_sink_mode),
// when bwd_dkdv_kernel's grid of 64-key blocks would not give every CU a workgroup (an 8-head
// shard of a GPT-OSS layer: 64 blocks of 4096 keys).  There its twice as many workgroups, each with
// fewer rows and no idle waves, finish sooner (measured on MI355X: 19.5 us against 29.5 us at
// L = 4096, W = 128, 8 heads).  On a full chip of 64-key workgroups bwd_dkdv_kernel is faster (its
// two key halves share each staged tile), as for full causal and long windows.
static bool dkdv4_eligible(const Args& a, int D) {
  return D <= 64 && a.G % 4 == 0 && a.W >= 1 && a.W <= 512 && (a.nsp == 0 || (a.sink_dq && a.n_chunks == 0)) &&
         int64_t(a.B) * a.Hkv * ((a.L + kKvKeys - 1) / kKvKeys) <= device_cus();
}

// The D = 64 dK/dV kernel with its K/V operands in LDS (three workgroups per CU instead of two)
// pays on grids of many short workgroups: windows up to 512 keys and at least six workgroups per
// CU.  Measured on MI355X (Hq = 64 or 32, D = 64): 4096 workgroups at W = 128 (L = 32768) 247
// against 272 us, at W = 512 666 against 695 us; 2048 workgroups (B = 4, G = 4) 67 against 75 us.
// With fewer workgroups the last, partly filled round of three per CU costs more than the extra
// workgroup gains (1024 at W = 128: 69 against 64 us; 512: 37 against 35 us), and the long sweeps
// of full causal attention are slower with the extra LDS reads (936 against 843 us at Hkv = 4).
static bool dkdv_kvl_pays(const Args& a, int grid) {
  return a.W <= 512 && grid >= 6 * device_cus();
}

// Waves (query-head slots) per workgroup of bwd_dkdv4_kernel: its grid is at most two 32-key
// workgroups per CU, so with a large KV group (an MQA layer, or a KV-group shard) four waves leave
// SIMDs idle and each wave sweeps G / 4 heads.  Up to two waves per SIMD, the workgroup takes 8
// waves (or 16 at D = 16, whose 122 VGPRs allow four per SIMD) when G is a multiple of that.
static int dkdv4_waves(const Args& a, int D, int grid) {
  const int waves = 8 * device_cus();  // two per SIMD
  if (D == 16 && a.G % 16 == 0 && grid * 16 <= waves) return 16;
  if (a.G % 8 == 0 && grid * 8 <= waves) return 8;
  return 4;
}

template <typename E, int D>
static hipError_t launch_dkdv_d(const Args& a, hipStream_t stream) {
  Args ad = a;
  // the in-kernel fold finds the dQ slots by the dQ grid (and sizes its run list in LDS by it)
  if (a.sink_dq) ad.dq_wgs = a.dq_slide ? (a.G / 8) * a.slide_ncu : dq_grid<E, D, true>(a);
  hipError_t e;
  bool folded;
  if constexpr (D <= 64) {
    if (dkdv4_eligible(a, D)) {
      ad.n_kblocks = (a.L + 31) / 32;  // 32-key blocks
      const int grid = a.B * a.Hkv * ad.n_kblocks;
      const int nw = dkdv4_waves(a, D, grid);
      if constexpr (D == 16) {
        if (nw == 16) {
          hipLaunchKernelGGL((bwd_dkdv4_kernel<E, D, 16>), dim3(grid), dim3(1024), 0, stream, ad);
          folded = dkdv4_folds_in_kernel(ad, D, dkdv4_lds_elems<D, 16>());
        }
      }
      if (nw == 8) {
        hipLaunchKernelGGL((bwd_dkdv4_kernel<E, D, 8>), dim3(grid), dim3(512), 0, stream, ad);
        folded = dkdv4_folds_in_kernel(ad, D, dkdv4_lds_elems<D, 8>());
      } else if (nw == 4) {
        hipLaunchKernelGGL((bwd_dkdv4_kernel<E, D>), dim3(grid), dim3(256), 0, stream, ad);
        folded = dkdv4_folds_in_kernel(ad, D, dkdv4_lds_elems<D>());
      }
      e = hipGetLastError();
    } else {
      const int per_kv = a.vl_kblocks ? a.vl_kblocks : a.B * a.n_kblocks;  // regular workgroups per KV head
      const int grid = a.n_chunk_wgs + a.Hkv * per_kv;
      bool kvl = false;
      if constexpr (D == 64) kvl = dkdv_kvl_pays(a, grid);
      if constexpr (D == 64) {
        if (kvl) hipLaunchKernelGGL((bwd_dkdv_kernel<E, D, true>), dim3(grid), dim3(256), 0, stream, ad);
      }
      if (!kvl) hipLaunchKernelGGL((bwd_dkdv_kernel<E, D>), dim3(grid), dim3(256), 0, stream, ad);
      e = hipGetLastError();
      folded = dkdv_folds_in_kernel(ad, D, kvl);
    }
  } else {
    const int per_kv = a.vl_kblocks ? a.vl_kblocks : a.B * a.n_kblocks;
    hipLaunchKernelGGL((bwd_dkdv_kernel<E, D>), dim3(a.n_chunk_wgs + a.Hkv * per_kv), dim3(256), 0, stream, ad);
    e = hipGetLastError();
    folded = dkdv_folds_in_kernel(ad, D, false);
  }
  // the sink keys are folded inside the dK/dV kernel or by a launch of their own
  if (e != hipSuccess || a.nsp == 0 || folded) return e;
  const int64_t n = int64_t(a.B) * a.Hkv * min(a.S, kKvKeys * a.nsp);  // one workgroup per sink key
  hipLaunchKernelGGL((bwd_sink_fold_kernel<E, D>), dim3(unsigned(n)), dim3(256), 0, stream, ad);
  return hipGetLastError();
}

#define FA_DISPATCH_D(FN, E, D, ...)                          \
  switch (D) {                                                \
    case 16: return FN<E, 16>(__VA_ARGS__);                   \
    case 32: return FN<E, 32>(__VA_ARGS__);                   \
    case 64: return FN<E, 64>(__VA_ARGS__);                   \
    case 128: return FN<E, 128>(__VA_ARGS__);                 \
  }                                                           \
  return hipErrorInvalidValue;

template <typename E>
static hipError_t dq_e(const Args& a, int D, int hpw, hipStream_t s) { FA_DISPATCH_D(launch_dq_d, E, D, a, hpw, s) }
template <typename E>
static hipError_t dkdv_e(const Args& a, int D, hipStream_t s) { FA_DISPATCH_D(launch_dkdv_d, E, D, a, s) }

hipError_t launch_bwd_dq(const Args& a, int dtype, int D, int hpw, hipStream_t s) {
  return dtype == 1 ? dq_e<BF16>(a, D, hpw, s) : dq_e<F16>(a, D, hpw, s);
}
hipError_t launch_bwd_dkdv(const Args& a, int dtype, int D, hipStream_t s) {
  return dtype == 1 ? dkdv_e<BF16>(a, D, s) : dkdv_e<F16>(a, D, s);
}
hipError_t launch_bwd_sink_logits(const Args& a, hipStream_t s) {
  hipLaunchKernelGGL(bwd_sink_logit_kernel, dim3(a.Hq), dim3(256), 0, s, a);
  return hipGetLastError();
}
#endif  // FA_BWD_WIDE_TU


}  // namespace fa
