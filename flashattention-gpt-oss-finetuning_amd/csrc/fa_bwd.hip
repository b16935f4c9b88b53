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
// Three launches:
//  1. bwd_dq_kernel (query-major, same tiling as the forward): computes delta for its rows
//     (stored in the workspace) and dQ over the sink + window key blocks.
//  2. bwd_dkdv_kernel (key-major): a workgroup owns 32 keys of one KV head and sweeps the
//     (query head, 32-row query block) pairs that can see those keys; its 4 waves split that
//     sweep and their fp32 partial sums are added in LDS in a fixed order, so the result is
//     deterministic.  The sweep of a key block is bounded by the window: rows
//     [k0, k0 + 31 + W).  Sink keys are also seen by every later row; those rows are split
//     into chunks of `chunk_rows` handled by extra workgroups of the same kernel that write
//     fp32 partial sums to the workspace (the reference instead loops one program over all
//     of L for a sink block, benchmark_backward_speed.py:432-438).
//  3. bwd_sink_finalize_kernel: adds the partial sums of the sink blocks in a fixed order and
//     writes those dK/dV rows (only when some sink rows were chunked).
#include "fa_args.h"
#include "fa_common.h"

namespace fa {

// ---------------------------------------------------------------------------------------------
// dQ (query-major).  Per wave: 32 rows x HPW heads.  Per 32-key step, with S^T = K Q^T and
// dP^T = V dO^T in C layout (lane = query row), P and dS are per-lane elementwise, and
// dQ^T += K^T dS^T takes dS^T straight from registers while K^T comes from LDS.
// ---------------------------------------------------------------------------------------------
template <typename E, int D, int HPW>
__global__ __launch_bounds__(256) void bwd_dq_kernel(const Args a) {
  constexpr int BN = 64;
  constexpr int KS = D / 16;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int KROW = D + 8;
  constexpr int TROW = BN + 8;
  constexpr int BUF = 2 * BN * KROW + D * TROW;  // K, V row-major + K^T permuted
  constexpr int NK = (BN * D / 8 + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * BUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, hf = lane >> 5;

  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = tile % a.n_qtiles;
  const int hg = tile / a.n_qtiles;
  const int hwg = HPW * a.wh;
  const int groups_per_batch = a.Hq / hwg;
  const int b = hg / groups_per_batch;
  const int h0 = (hg % groups_per_batch) * hwg;
  const int kvh = h0 / a.G;
  const int BM = 32 * a.wq;
  const int q0 = qt * BM;
  const int qw = q0 + 32 * (wave % a.wq);
  const int hw = h0 + HPW * (wave / a.wq);
  const int q = qw + r32;
  const bool wave_active = qw < a.L;
  const int L = a.L, W = a.W, S = a.S;

  // Row operands and row statistics.
  u32x4 qf[HPW][KS], dof[HPW][KS];
  float lse2[HPW], delta[HPW];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    const char* qp = reinterpret_cast<const char*>(a.q) +
                     2 * (int64_t(b) * a.sq[0] + int64_t(hw + h) * a.sq[1] + int64_t(q) * a.sq[2]);
    const char* dop = reinterpret_cast<const char*>(a.dout) +
                      2 * (int64_t(b) * a.sdo[0] + int64_t(hw + h) * a.sdo[1] + int64_t(q) * a.sdo[2]);
    const char* op = reinterpret_cast<const char*>(a.o) +
                     2 * (int64_t(b) * a.so[0] + int64_t(hw + h) * a.so[1] + int64_t(q) * a.so[2]);
    float dsum = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d = hf * (D / 2) + 8 * ks;
      u32x4 qv = zero16(), dv = zero16(), ov = zero16();
      if (q < L) {
        qv = ld16(qp + 2 * d);
        dv = ld16(dop + 2 * d);
        ov = ld16(op + 2 * d);
      }
      qf[h][ks] = qv ^ a.qsign;
      dof[h][ks] = dv;
      dsum += dot8<E>(dv, ov);
    }
    delta[h] = dsum + xor32(dsum);
    lse2[h] = __builtin_inff();
    if (q < L) {
      lse2[h] = a.lse[int64_t(b) * a.slse[0] + int64_t(hw + h) * a.slse[1] + int64_t(q) * a.slse[2]] * kLog2e;
      if (hf == 0) a.delta[(int64_t(b) * a.Hq + hw + h) * a.Lp + q] = delta[h];
    }
  }

  f32x16 acc[HPW][DB];
#pragma unroll
  for (int h = 0; h < HPW; ++h)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[h][db] = f32x16{};

  const QPlan plan = qplan(q0, BM, L, W, S);

  const char* kbase = reinterpret_cast<const char*>(a.k) + 2 * (int64_t(b) * a.sk[0] + int64_t(kvh) * a.sk[1]);
  const char* vbase = reinterpret_cast<const char*>(a.v) + 2 * (int64_t(b) * a.sv[0] + int64_t(kvh) * a.sv[1]);

  u32x4 kreg[NK], vreg[NK];
  auto gload = [&](int kb) {
#pragma unroll
    for (int it = 0; it < NK; ++it) {
      const int c = tid + 256 * it;
      const int row = c / (D / 8), col = c % (D / 8);
      u32x4 kv = zero16(), vv = zero16();
      if (c < BN * D / 8 && kb + row < L) {
        kv = ld16(kbase + 2 * (int64_t(kb + row) * a.sk[2] + 8 * col));
        vv = ld16(vbase + 2 * (int64_t(kb + row) * a.sv[2] + 8 * col));
      }
      kreg[it] = kv;
      vreg[it] = vv;
    }
  };
  auto sstore = [&](int buf) {
    uint16_t* Kl = lds + buf * BUF;
    uint16_t* Vl = Kl + BN * KROW;
#pragma unroll
    for (int it = 0; it < NK; ++it) {
      const int c = tid + 256 * it;
      const int row = c / (D / 8), col = c % (D / 8);
      if (c < BN * D / 8) {
        st16(Kl + row * KROW + 8 * col, kreg[it]);
        st16(Vl + row * KROW + 8 * col, vreg[it]);
      }
    }
  };
  auto tstore = [&](int buf) {
    // K^T (permuted key order) from the K rows just written to LDS: thread tid < 2*D owns one
    // unit of 4 keys x 8 head-dim indices.
    const uint16_t* Kl = lds + buf * BUF;
    uint16_t* Tl = lds + buf * BUF + 2 * BN * KROW;
    if (tid < 2 * D) {
      const int dc = tid % (D / 8), kq = tid / (D / 8);
      u32x4 rows[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) rows[r] = *reinterpret_cast<const u32x4*>(Kl + (4 * kq + r) * KROW + 8 * dc);
      u32x2 cols[8];
      transpose4x8(rows, cols);
      const int pos = perm_pos(4 * kq);
#pragma unroll
      for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x2*>(Tl + (8 * dc + i) * TROW + pos) = cols[i];
    }
  };

  gload(qplan_block(plan, 0));
  sstore(0);
  __syncthreads();
  tstore(0);
  __syncthreads();

  for (int i = 0; i < plan.nb; ++i) {
    const int kb = qplan_block(plan, i);
    const bool more = i + 1 < plan.nb;
    if (more) gload(qplan_block(plan, i + 1));
    if (wave_active) {
      const uint16_t* Kl = lds + (i & 1) * BUF;
      const uint16_t* Vl = Kl + BN * KROW;
      const uint16_t* Tl = Kl + 2 * BN * KROW;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int ks0 = kb + 32 * sb;
        if (!wave_needs(ks0, qw, L, W, S)) continue;
        f32x16 s[HPW], dp[HPW];
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
          s[h] = f32x16{};
          dp[h] = f32x16{};
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int off = (32 * sb + r32) * KROW + hf * (D / 2) + 8 * ks;
          const u32x4 kf = *reinterpret_cast<const u32x4*>(Kl + off);
          const u32x4 vf = *reinterpret_cast<const u32x4*>(Vl + off);
#pragma unroll
          for (int h = 0; h < HPW; ++h) {
            s[h] = E::mfma(kf, qf[h][ks], s[h]);
            dp[h] = E::mfma(vf, dof[h][ks], dp[h]);
          }
        }
        const bool full = tile_full(ks0, qw, W, S);
        u32x4 dsb[HPW][2];
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
          float ds[16];
          const int kl = ks0 + 4 * hf;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int off = 8 * (e / 4) + (e % 4);
            float p = fast_exp2(fmaf(s[h][e], a.c, -lse2[h]));
            if (!full && !allowed(q - kl - off, kl + off, W, S)) p = 0.f;
            ds[e] = p * (dp[h][e] - delta[h]);
          }
          dsb[h][0] = pack8<E>(ds);
          dsb[h][1] = pack8<E>(ds + 8);
        }
        const int trow = sigma32(r32);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            u32x4 kt = zero16();
            if (D >= 32 || trow < D)
              kt = *reinterpret_cast<const u32x4*>(Tl + (32 * db + trow) * TROW + 32 * sb + 16 * t + 8 * hf);
#pragma unroll
            for (int h = 0; h < HPW; ++h) acc[h][db] = E::mfma(kt, dsb[h][t], acc[h][db]);
          }
        }
      }
    }
    if (more) {
      sstore((i + 1) & 1);
      __syncthreads();
      tstore((i + 1) & 1);
    }
    __syncthreads();
  }

  if (!wave_active || q >= L) return;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    char* dqp = reinterpret_cast<char*>(a.dq) +
                2 * (int64_t(b) * a.sdq[0] + int64_t(hw + h) * a.sdq[1] + int64_t(q) * a.sdq[2]);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      if (D == 16 && hf == 1) continue;
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = acc[h][db][e] * a.scale;
      const int d0 = 32 * db + (D >= 32 ? 16 * hf : 0);
      st16(dqp + 2 * d0, pack8<E>(v));
      st16(dqp + 2 * (d0 + 8), pack8<E>(v + 8));
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dK / dV (key-major).  Per (query head, 32-row block): S = Q K^T and dP = dO V^T in C layout
// (lane = key column, 16 query rows per lane), then dV^T += dO^T P and dK^T += Q^T dS with
// P/dS straight from registers and dO^T/Q^T staged per wave in LDS (permuted row order).
// ---------------------------------------------------------------------------------------------
template <typename E, int D>
__global__ __launch_bounds__(256) void bwd_dkdv_kernel(const Args a) {
  constexpr int KS = D / 16;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  constexpr int TROW = 32 + 8;                    // transposed tile row stride (elements)
  constexpr int TILE = D * TROW;                  // one [D][32] transposed tile
  constexpr int WAVE_LDS = 2 * TILE;              // Q^T and dO^T per wave (elements)
  constexpr int RED_FLOATS = 3 * DB * 16 * 64;    // partial sums of waves 1..3
  constexpr int LDS_ELEMS = (4 * WAVE_LDS > 2 * RED_FLOATS) ? 4 * WAVE_LDS : 2 * RED_FLOATS;  // uint16 units
  constexpr int NU = (D + 63) / 64;               // transposed-load units per lane
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, hf = lane >> 5;
  const int L = a.L, W = a.W, S = a.S, G = a.G;

  // Which key block and which query rows this workgroup owns.
  int id = xcd_remap(blockIdx.x, gridDim.x);
  int b, kvh, kblk, slot = -1, qlo, qhi;
  bool to_partial;
  if (id < a.n_chunk_wgs) {
    const int c = id % a.n_chunks;
    int t = id / a.n_chunks;
    kblk = t % a.nsp;
    t /= a.nsp;
    kvh = t % a.Hkv;
    b = t / a.Hkv;
    qlo = kv_chunk_lo(kblk, c, a.chunk_rows, L, W);
    qhi = kv_chunk_hi(c, a.chunk_rows, L);
    slot = c;
    to_partial = true;
  } else {
    id -= a.n_chunk_wgs;
    kblk = id % a.n_kblocks;
    const int t = id / a.n_kblocks;
    kvh = t % a.Hkv;
    b = t / a.Hkv;
    qlo = 32 * kblk;
    qhi = kv_window_end(kblk, L, W);
    to_partial = kblk < a.nsp;
    slot = a.n_chunks;
  }
  const int ks0 = 32 * kblk;
  const int key = ks0 + r32;  // this lane's key column

  // K^T / V^T operands (B of S = Q K^T and dP = dO V^T): lane (key, hf) holds head-dim slice
  // [hf*D/2 + 8ks, +8).
  u32x4 kf[KS], vf[KS];
  {
    const char* kp = reinterpret_cast<const char*>(a.k) +
                     2 * (int64_t(b) * a.sk[0] + int64_t(kvh) * a.sk[1] + int64_t(key) * a.sk[2]);
    const char* vp = reinterpret_cast<const char*>(a.v) +
                     2 * (int64_t(b) * a.sv[0] + int64_t(kvh) * a.sv[1] + int64_t(key) * a.sv[2]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d = hf * (D / 2) + 8 * ks;
      kf[ks] = key < L ? ld16(kp + 2 * d) : zero16();
      vf[ks] = key < L ? ld16(vp + 2 * d) : zero16();
    }
  }

  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }

  const int qb_lo = qlo / 32;
  const int n_qb = qhi > qlo ? (qhi + 31) / 32 - qb_lo : 0;
  const int n_it = G * n_qb;
  uint16_t* QT = lds + wave * WAVE_LDS;
  uint16_t* DT = QT + TILE;

  for (int it = wave; it < n_it; it += 4) {
    const int hl = it / n_qb;
    const int qb = qb_lo + it % n_qb;
    const int h = kvh * G + hl;
    const int qr0 = 32 * qb;
    const int64_t qoff = int64_t(b) * a.sq[0] + int64_t(h) * a.sq[1];
    const int64_t dooff = int64_t(b) * a.sdo[0] + int64_t(h) * a.sdo[1];
    const char* qbase = reinterpret_cast<const char*>(a.q) + 2 * qoff;
    const char* dobase = reinterpret_cast<const char*>(a.dout) + 2 * dooff;

    // Stage Q^T and dO^T of rows [qr0, qr0+32) in this wave's LDS (permuted row order).
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int unit = lane + 64 * u;
      if (unit < D) {  // D units: 8 row quads x D/8 head-dim chunks
        const int dc = unit % (D / 8), rq = unit / (D / 8);
        u32x4 qr[4], dr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = qr0 + 4 * rq + r;
          qr[r] = zero16();
          dr[r] = zero16();
          if (row < L) {
            qr[r] = ld16(qbase + 2 * (int64_t(row) * a.sq[2] + 8 * dc));
            dr[r] = ld16(dobase + 2 * (int64_t(row) * a.sdo[2] + 8 * dc));
          }
        }
        u32x2 qc[8], dc8[8];
        transpose4x8(qr, qc);
        transpose4x8(dr, dc8);
        const int pos = perm_pos(4 * rq);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          *reinterpret_cast<u32x2*>(QT + (8 * dc + i) * TROW + pos) = qc[i];
          *reinterpret_cast<u32x2*>(DT + (8 * dc + i) * TROW + pos) = dc8[i];
        }
      }
    }

    // Row operands Q, dO (A of S and dP): lane (row qr0 + r32, hf).
    const int arow = qr0 + r32;
    u32x4 qa[KS], da[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d = hf * (D / 2) + 8 * ks;
      qa[ks] = zero16();
      da[ks] = zero16();
      if (arow < L) {
        qa[ks] = ld16(qbase + 2 * (int64_t(arow) * a.sq[2] + d));
        da[ks] = ld16(dobase + 2 * (int64_t(arow) * a.sdo[2] + d));
      }
      qa[ks] ^= a.qsign;
    }
    // Row statistics of the 16 rows this lane holds in C layout: qr0 + 8j + 4hf + (0..3).
    float l2[16], dl[16];
    const float* lsep = a.lse + int64_t(b) * a.slse[0] + int64_t(h) * a.slse[1];
    const float* dlp = a.delta + (int64_t(b) * a.Hq + h) * a.Lp;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r0 = qr0 + 8 * j + 4 * hf;
      const f32x4 dq4 = *reinterpret_cast<const f32x4*>(dlp + r0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + e;
        l2[4 * j + e] = row < L ? lsep[int64_t(row) * a.slse[2]] * kLog2e : __builtin_inff();
        dl[4 * j + e] = row < L ? dq4[e] : 0.f;
      }
    }

    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      s = E::mfma(qa[ks], kf[ks], s);
      dp = E::mfma(da[ks], vf[ks], dp);
    }
    // Rows outside [qlo, qhi) belong to another workgroup; rows/keys outside the mask are 0.
    const bool full = (qr0 >= qlo) && (qr0 + 32 <= qhi) && tile_full(ks0, qr0, W, S);
    float p[16], ds[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = qr0 + 8 * (e / 4) + 4 * hf + (e % 4);
      float pe = fast_exp2(fmaf(s[e], a.c, -l2[e]));
      if (!full && !(row >= qlo && row < qhi && allowed(row - key, key, W, S))) pe = 0.f;
      p[e] = pe;
      ds[e] = pe * (dp[e] - dl[e]);
    }
    const u32x4 pb0 = pack8<E>(p), pb1 = pack8<E>(p + 8);
    const u32x4 sb0 = pack8<E>(ds), sb1 = pack8<E>(ds + 8);
    const int trow = sigma32(r32);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        u32x4 dt = zero16(), qt = zero16();
        if (D >= 32 || trow < D) {
          const int off = (32 * db + trow) * TROW + 16 * t + 8 * hf;
          dt = *reinterpret_cast<const u32x4*>(DT + off);
          qt = *reinterpret_cast<const u32x4*>(QT + off);
        }
        dv[db] = E::mfma(dt, t ? pb1 : pb0, dv[db]);
        dk[db] = E::mfma(qt, t ? sb1 : sb0, dk[db]);
      }
    }
  }

  // Fixed-order reduction of the 4 waves' partial sums (wave 0 + 1 + 2 + 3), dK then dV.
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    f32x16* x = part ? dv : dk;
    __syncthreads();
    if (wave > 0) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[(((wave - 1) * DB + db) * 16 + e) * 64 + lane] = x[db][e];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e)
#pragma unroll
          for (int w = 0; w < 3; ++w) x[db][e] += red[((w * DB + db) * 16 + e) * 64 + lane];
    }
  }
  if (wave != 0) return;

  // Lane (key, hf) owns head-dim indices 32db + 16hf + e (D == 16: hf == 0 only).
  if (to_partial) {
    float* pk = a.partial + ((((int64_t(b) * a.Hkv + kvh) * a.nsp + kblk) * (a.n_chunks + 1) + slot) * 2) * 32 * D;
    float* pv = pk + 32 * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      if (D == 16 && hf == 1) continue;
      const int d0 = 32 * db + (D >= 32 ? 16 * hf : 0);
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        *reinterpret_cast<f32x4*>(pk + r32 * D + d0 + 4 * e4) =
            f32x4{dk[db][4 * e4], dk[db][4 * e4 + 1], dk[db][4 * e4 + 2], dk[db][4 * e4 + 3]};
        *reinterpret_cast<f32x4*>(pv + r32 * D + d0 + 4 * e4) =
            f32x4{dv[db][4 * e4], dv[db][4 * e4 + 1], dv[db][4 * e4 + 2], dv[db][4 * e4 + 3]};
      }
    }
    return;
  }
  if (key >= L) return;
  char* dkp = reinterpret_cast<char*>(a.dk) +
              2 * (int64_t(b) * a.sdk[0] + int64_t(kvh) * a.sdk[1] + int64_t(key) * a.sdk[2]);
  char* dvp = reinterpret_cast<char*>(a.dv) +
              2 * (int64_t(b) * a.sdv[0] + int64_t(kvh) * a.sdv[1] + int64_t(key) * a.sdv[2]);
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    if (D == 16 && hf == 1) continue;
    float kv[16], vv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      kv[e] = dk[db][e] * a.scale;
      vv[e] = dv[db][e];
    }
    const int d0 = 32 * db + (D >= 32 ? 16 * hf : 0);
    st16(dkp + 2 * d0, pack8<E>(kv));
    st16(dkp + 2 * (d0 + 8), pack8<E>(kv + 8));
    st16(dvp + 2 * d0, pack8<E>(vv));
    st16(dvp + 2 * (d0 + 8), pack8<E>(vv + 8));
  }
}

// ---------------------------------------------------------------------------------------------
// Sink finalize: dK/dV rows of the chunked sink blocks = fixed-order sum of their partials.
// One thread per (b, kvh, block, row, head-dim index).
// ---------------------------------------------------------------------------------------------
template <typename E, int D>
__global__ __launch_bounds__(256) void bwd_sink_finalize_kernel(const Args a) {
  const int64_t n = int64_t(a.B) * a.Hkv * a.nsp * 32 * D;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int d = int(i % D);
  const int row = int((i / D) % 32);
  const int64_t blk = i / (int64_t(32) * D);  // (b*Hkv + kvh)*nsp + kblk
  const int kblk = int(blk % a.nsp);
  const int kvh = int((blk / a.nsp) % a.Hkv);
  const int b = int(blk / (int64_t(a.nsp) * a.Hkv));
  const int key = 32 * kblk + row;
  if (key >= a.L) return;
  const float* base = a.partial + blk * (a.n_chunks + 1) * 2 * 32 * D + row * D + d;
  float sk = 0.f, sv = 0.f;
  for (int s = 0; s <= a.n_chunks; ++s) {
    sk += base[int64_t(s) * 2 * 32 * D];
    sv += base[int64_t(s) * 2 * 32 * D + 32 * D];
  }
  sk *= a.scale;
  uint16_t* dkp = reinterpret_cast<uint16_t*>(a.dk) + int64_t(b) * a.sdk[0] + int64_t(kvh) * a.sdk[1] +
                  int64_t(key) * a.sdk[2] + d;
  uint16_t* dvp = reinterpret_cast<uint16_t*>(a.dv) + int64_t(b) * a.sdv[0] + int64_t(kvh) * a.sdv[1] +
                  int64_t(key) * a.sdv[2] + d;
  const uint32_t pk = E::pack2(sk, sv);
  *dkp = uint16_t(pk);
  *dvp = uint16_t(pk >> 16);
}

// ---------------------------------------------------------------------------------------------
template <typename E, int D>
static hipError_t launch_dq_d(const Args& a, int hpw, hipStream_t stream) {
  const int groups = a.B * a.Hq / (hpw * a.wh);
  const dim3 grid(a.n_qtiles * groups), block(256);
  if (hpw == 2) hipLaunchKernelGGL((bwd_dq_kernel<E, D, 2>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((bwd_dq_kernel<E, D, 1>), grid, block, 0, stream, a);
  return hipGetLastError();
}

template <typename E, int D>
static hipError_t launch_dkdv_d(const Args& a, hipStream_t stream) {
  const dim3 grid(a.n_chunk_wgs + a.B * a.Hkv * a.n_kblocks), block(256);
  hipLaunchKernelGGL((bwd_dkdv_kernel<E, D>), grid, block, 0, stream, a);
  return hipGetLastError();
}

template <typename E, int D>
static hipError_t launch_fin_d(const Args& a, hipStream_t stream) {
  const int64_t n = int64_t(a.B) * a.Hkv * a.nsp * 32 * D;
  const dim3 grid(unsigned((n + 255) / 256)), block(256);
  hipLaunchKernelGGL((bwd_sink_finalize_kernel<E, D>), grid, block, 0, stream, a);
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
template <typename E>
static hipError_t fin_e(const Args& a, int D, hipStream_t s) { FA_DISPATCH_D(launch_fin_d, E, D, a, s) }

hipError_t launch_bwd_dq(const Args& a, int dtype, int D, int hpw, hipStream_t s) {
  return dtype == 1 ? dq_e<BF16>(a, D, hpw, s) : dq_e<F16>(a, D, hpw, s);
}
hipError_t launch_bwd_dkdv(const Args& a, int dtype, int D, hipStream_t s) {
  return dtype == 1 ? dkdv_e<BF16>(a, D, s) : dkdv_e<F16>(a, D, s);
}
hipError_t launch_bwd_sink_finalize(const Args& a, int dtype, int D, hipStream_t s) {
  return dtype == 1 ? fin_e<BF16>(a, D, s) : fin_e<F16>(a, D, s);
}

}  // namespace fa
