// fa_f32.hip - float32 inputs: forward and backward on the fp32 matrix instruction.
//
// The reference's autograd Function takes float32 q/k/v as well as 16-bit ones
// (flash_attention_gpt_oss.py:356-357: o = empty_like(q); benchmark_backward_speed.py:28-37:
// dtype "fp32").  These kernels compute that case in float32 throughout: every product runs on
// v_mfma_f32_32x32x2_f32 (exact fp32 products, fp32 sums), P and dS stay fp32, and q, k, v, o,
// dq, dk, dv are fp32 tensors.  The mathematics, masks, visit order of key blocks, workspace row
// statistics and the sink-key partial sums follow the 16-bit kernels (fa_fwd.hip, fa_bwd.hip).
//
// The instruction: a wave64 multiplies a 32x2 A tile by a 2x32 B tile into a 32x32 fp32 C tile;
// lane l (r = l % 32, h = l / 32) supplies A[r][h] and B[h][r] and holds C[crow(i, h)][r] for
// i = 0..15, crow(i, h) = 8 (i / 4) + 4 h + i % 4 -- the C layout of the 32x32x16 16-bit form.
// Two consequences, as in the 16-bit kernels:
//  * a product over a head dim of D runs as D / 2 instructions; in step t lane half h supplies
//    head-dim index h D / 2 + t, so each lane reads one contiguous half row;
//  * a C tile feeds the next product as its B operand unchanged: in step t the reduction index
//    of lane half h is crow(t, h), which is register t of every lane.
// Each workgroup is one wave: 32 query rows of one head (forward, dQ) or 32 keys of one KV head
// (dK/dV).  Operands come straight from memory (L1/L2), no LDS.
#include "fa_args.h"
#include "fa_common.h"

namespace fa {

namespace {

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int crow(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }
__device__ __forceinline__ f32x4 ld4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4f(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ float other_half(float x) { return __shfl_xor(x, 32); }

// Key tiles of 32 that rows [q0, q0 + 32) of a sequence of L rows visit: the sink tiles [0, nsink)
// (keys below S that lie before the window tiles) and the window tiles [ws, we).
struct Plan32 {
  int nsink, ws, we;
};
__device__ __forceinline__ Plan32 plan32(int q0, int L, int W, int S) {
  Plan32 p;
  const int q_end = min(q0 + 32, L);
  const int wlo = max(0, q0 - W + 1);  // first key in any row's window
  p.ws = wlo / 32;
  p.we = q_end > wlo ? (q_end - 1) / 32 + 1 : p.ws;
  p.nsink = (min(S, 32 * p.ws) + 31) / 32;
  return p;
}
__device__ __forceinline__ int plan32_tile(const Plan32& p, int i) { return i < p.nsink ? i : p.ws + (i - p.nsink); }
__device__ __forceinline__ bool allowed32(int q, int k, int W, int S) { return k <= q && (q - k < W || k < S); }

// One fp32 half row (D / 2 values starting at column h D / 2) of row `row` of a [rows][stride]
// slice, times `mul`; zeros for rows past L.
template <int D>
__device__ __forceinline__ void load_half_row(const float* base, int64_t stride, int row, int L, int h, float mul,
                                              float (&out)[D / 2]) {
  const float* p = base + int64_t(row) * stride + h * (D / 2);
#pragma unroll
  for (int u = 0; u < D / 8; ++u) {
    const f32x4 x = row < L ? ld4f(p + 4 * u) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) out[4 * u + j] = x[j] * mul;
  }
}

// ---------------------------------------------------------------------------------------------
// Forward: O = softmax(mask(s)) V with s = scale q.k, online softmax in the log2 domain (q is
// pre-multiplied by scale * log2(e)).  Grid (row tiles, Hq, B), one wave each.
// ---------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64) void fwd32_kernel(const Args a) {
  constexpr int HD = D / 2;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  const int lane = threadIdx.x, r = lane & 31, h = lane >> 5;
  const int hq = blockIdx.y, b = blockIdx.z;
  const Seq sq = seq_of(a, b);
  const int L = sq.L, q0 = 32 * int(blockIdx.x);
  if (q0 >= L) return;
  const int kvh = hq / a.G, W = a.W, S = a.S;
  const float* Q = static_cast<const float*>(a.q) + slice_off(a.sq, b, hq, sq.row);
  const float* K = static_cast<const float*>(a.k) + slice_off(a.sk, b, kvh, sq.row);
  const float* V = static_cast<const float*>(a.v) + slice_off(a.sv, b, kvh, sq.row);
  const int q = q0 + r;
  float qf[HD];
  load_half_row<D>(Q, a.sq[2], q, L, h, a.scale * kLog2e, qf);

  float m = kNegInf, lsum = 0.f;
  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
  const Plan32 pl = plan32(q0, L, W, S);
  const int nt = pl.nsink + (pl.we - pl.ws);
  for (int it = 0; it < nt; ++it) {
    const int ks0 = 32 * plan32_tile(pl, it);
    // S^T = K Q^T (keys x queries): lane (r, h) supplies K[ks0 + r][h HD + t]
    float kf[HD];
    load_half_row<D>(K, a.sk[2], ks0 + r, L, h, 1.f, kf);
    f32x16 s = f32x16{};
#pragma unroll
    for (int t = 0; t < HD; ++t) s = mfma32(kf[t], qf[t], s);
    float mx = kNegInf;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = allowed32(q, ks0 + crow(i, h), W, S) ? s[i] : kNegInf;
      mx = fmaxf(mx, s[i]);
    }
    mx = fmaxf(mx, other_half(mx));
    const float mnew = fmaxf(m, mx);
    const float alpha = mnew == kNegInf ? 1.f : exp2f(m - mnew);
    const float ms = mnew == kNegInf ? 0.f : mnew;
    m = mnew;
    lsum *= alpha;
    float p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      p[i] = exp2f(s[i] - ms);
      lsum += p[i];
    }
    // O^T += V^T P^T: lane (r, h) supplies V[ks0 + crow(t, h)][32 db + r]
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      acc[db] *= alpha;
      const int d = 32 * db + r;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int kk = ks0 + crow(t, h);
        const float va = (d < D && kk < L) ? V[int64_t(kk) * a.sv[2] + d] : 0.f;
        acc[db] = mfma32(va, p[t], acc[db]);
      }
    }
  }
  float lt = lsum + other_half(lsum);
  float rs = 1.f;
  if (a.sink_logits) {  // the learned sink joins the denominator (as in fwd_kernel's epilogue)
    const float sl = a.sink_logits[hq] * kLog2e;
    const float mn = fmaxf(m, sl);
    rs = m == kNegInf ? 0.f : exp2f(m - mn);
    lt = lt * rs + exp2f(sl - mn);
    m = mn;
  }
  if (q >= L) return;
  const float inv = lt > 0.f ? rs / lt : 0.f;
  float* O = static_cast<float*>(a.o_out) + slice_off(a.so_out, b, hq, sq.row + q);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * db + 8 * j + 4 * h;
      if (d < D) st4f(O + d, f32x4{acc[db][4 * j] * inv, acc[db][4 * j + 1] * inv, acc[db][4 * j + 2] * inv,
                                   acc[db][4 * j + 3] * inv});
    }
  if (h == 0) a.lse_out[slice_off(a.slse, b, hq, sq.row + q)] = (m + log2f(lt)) * kLn2;
}

// ---------------------------------------------------------------------------------------------
// dQ: delta = rowsum(dO o O), P = exp2(s - lse2), dS = P (dP - delta), dQ = scale dS K.  Also
// stores the row statistics the dK/dV kernel reads (lse * log2(e), -delta per 32-row block, the
// layout of the 16-bit backward) and, with learned sinks, the per-block partials of their
// gradient.  Grid (row tiles, Hq, B), one wave each.
// ---------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64) void dq32_kernel(const Args a) {
  constexpr int HD = D / 2;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  const int lane = threadIdx.x, r = lane & 31, h = lane >> 5;
  const int hq = blockIdx.y, b = blockIdx.z;
  const Seq sq = seq_of(a, b);
  const int L = sq.L, q0 = 32 * int(blockIdx.x);
  if (q0 >= L) return;
  const int kvh = hq / a.G, W = a.W, S = a.S;
  const float* Q = static_cast<const float*>(a.q) + slice_off(a.sq, b, hq, sq.row);
  const float* K = static_cast<const float*>(a.k) + slice_off(a.sk, b, kvh, sq.row);
  const float* V = static_cast<const float*>(a.v) + slice_off(a.sv, b, kvh, sq.row);
  const float* O = static_cast<const float*>(a.o) + slice_off(a.so, b, hq, sq.row);
  const float* dO = static_cast<const float*>(a.dout) + slice_off(a.sdo, b, hq, sq.row);
  const int q = q0 + r;
  float qf[HD], dof[HD], of[HD];
  load_half_row<D>(Q, a.sq[2], q, L, h, a.scale * kLog2e, qf);
  load_half_row<D>(dO, a.sdo[2], q, L, h, 1.f, dof);
  load_half_row<D>(O, a.so[2], q, L, h, 1.f, of);
  float dsum = 0.f;
#pragma unroll
  for (int t = 0; t < HD; ++t) dsum = fmaf(dof[t], of[t], dsum);
  const float delta = dsum + other_half(dsum);
  const float lse2 = q < L ? a.lse[slice_off(a.slse, b, hq, sq.row + q)] * kLog2e : __builtin_inff();
  if (h == 0) {
    float* st = a.delta + ((int64_t(b) * a.Hq + hq) * (a.Lp / 32) + q0 / 32) * 64;
    st[r] = lse2;
    st[32 + r] = -delta;
  }
  if (a.sink_logits) {
    float v = (q < L && h == 0) ? exp2f(a.sink_logits[hq] * kLog2e - lse2) * delta : 0.f;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) a.dsink_part[(int64_t(b) * a.Hq + hq) * (a.Lp / 32) + q0 / 32] = -v;
  }

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
  const Plan32 pl = plan32(q0, L, W, S);
  const int nt = pl.nsink + (pl.we - pl.ws);
  for (int it = 0; it < nt; ++it) {
    const int ks0 = 32 * plan32_tile(pl, it);
    float kf[HD], vf[HD];
    load_half_row<D>(K, a.sk[2], ks0 + r, L, h, 1.f, kf);
    load_half_row<D>(V, a.sv[2], ks0 + r, L, h, 1.f, vf);
    // S^T = K Q^T and dP^T - delta = V dO^T - delta (keys x queries)
    f32x16 s = f32x16{}, dp;
#pragma unroll
    for (int i = 0; i < 16; ++i) dp[i] = -delta;
#pragma unroll
    for (int t = 0; t < HD; ++t) {
      s = mfma32(kf[t], qf[t], s);
      dp = mfma32(vf[t], dof[t], dp);
    }
    float ds[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = allowed32(q, ks0 + crow(i, h), W, S) ? exp2f(s[i] - lse2) : 0.f;
      ds[i] = p * dp[i];
    }
    // dQ^T += K^T dS^T: lane (r, h) supplies K[ks0 + crow(t, h)][32 db + r]
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int d = 32 * db + r;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int kk = ks0 + crow(t, h);
        const float ka = (d < D && kk < L) ? K[int64_t(kk) * a.sk[2] + d] : 0.f;
        acc[db] = mfma32(ka, ds[t], acc[db]);
      }
    }
  }
  if (q >= L) return;
  float* dQ = static_cast<float*>(a.dq) + slice_off(a.sdq, b, hq, sq.row + q);
  const float sc = a.scale;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * db + 8 * j + 4 * h;
      if (d < D) st4f(dQ + d, f32x4{acc[db][4 * j] * sc, acc[db][4 * j + 1] * sc, acc[db][4 * j + 2] * sc,
                                    acc[db][4 * j + 3] * sc});
    }
}

// Rows a key tile's regular workgroup covers: [ks0, kv32_row_end) -- every row whose window
// reaches a key of the tile (and the tile's own 32 rows, for its sink keys).  Sink keys are also
// seen by every later row; those rows go to chunk workgroups of kF32ChunkRows rows.
__device__ __forceinline__ int kv32_row_end(int ks0, int L, int W) { return min(L, ks0 + 31 + max(W, 1)); }

// ---------------------------------------------------------------------------------------------
// dK / dV: a wave owns 32 keys of one KV head and sweeps the (query head, 32-row block) items
// that can see them: dV^T += dO^T P, dK^T += Q^T dS (keys as the C columns).  Grid (items, Hkv,
// B): blockIdx.x < n_kblocks is key tile x with its window rows; the rest are chunk workgroups,
// (sink tile st, chunk c) = ((x - n_kblocks) % nsp, (x - n_kblocks) / nsp), with the rows past
// the window of sink tile st.  Sink tiles write fp32 partials to the workspace (slot 0: the
// regular rows, slot c + 1: chunk c); fold32_kernel adds them.
// ---------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64) void dkdv32_kernel(const Args a) {
  constexpr int HD = D / 2;
  constexpr int DB = D >= 32 ? D / 32 : 1;
  const int lane = threadIdx.x, r = lane & 31, h = lane >> 5;
  const int kvh = blockIdx.y, b = blockIdx.z;
  const Seq sq = seq_of(a, b);
  const int L = sq.L, W = a.W, S = a.S, G = a.G;
  int kt, chunk = -1;
  if (int(blockIdx.x) < a.n_kblocks) {
    kt = blockIdx.x;
  } else {
    const int x = blockIdx.x - a.n_kblocks;
    kt = x % a.nsp;
    chunk = x / a.nsp;
  }
  const int ks0 = 32 * kt;
  if (ks0 >= L) return;
  const int row_end = kv32_row_end(ks0, L, W);
  const bool split = ks0 < S && row_end < L && kt < a.nsp;  // a sink tile with rows past its window
  int lo, hi;
  if (chunk < 0) {
    lo = ks0;
    hi = row_end;
  } else {
    if (!split) return;  // (this tile's rows all lie in its window: no chunk rows)
    lo = row_end + chunk * a.chunk_rows;
    hi = min(L, lo + a.chunk_rows);
  }
  const int key = ks0 + r;
  const float c2 = a.scale * kLog2e;
  const float* K = static_cast<const float*>(a.k) + slice_off(a.sk, b, kvh, sq.row);
  const float* V = static_cast<const float*>(a.v) + slice_off(a.sv, b, kvh, sq.row);
  float kf[HD], vf[HD];
  load_half_row<D>(K, a.sk[2], key, L, h, 1.f, kf);
  load_half_row<D>(V, a.sv[2], key, L, h, 1.f, vf);
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }
  for (int g = 0; g < G && lo < hi; ++g) {
    const int hq = kvh * G + g;
    const float* Q = static_cast<const float*>(a.q) + slice_off(a.sq, b, hq, sq.row);
    const float* dO = static_cast<const float*>(a.dout) + slice_off(a.sdo, b, hq, sq.row);
    const float* stat = a.delta + (int64_t(b) * a.Hq + hq) * (a.Lp / 32) * 64;
    for (int qr0 = lo / 32 * 32; qr0 < hi; qr0 += 32) {
      // S = Q K^T and dP - delta = dO V^T - delta (queries x keys): lane (r, h) supplies row
      // qr0 + r of Q (times scale log2 e) and of dO
      float qa[HD], da[HD];
      load_half_row<D>(Q, a.sq[2], qr0 + r, L, h, c2, qa);
      load_half_row<D>(dO, a.sdo[2], qr0 + r, L, h, 1.f, da);
      const float* st = stat + (qr0 / 32) * 64;
      float l2[16];
      f32x16 s = f32x16{}, dp;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 lv = ld4f(st + 8 * j + 4 * h), nv = ld4f(st + 32 + 8 * j + 4 * h);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          l2[4 * j + i] = lv[i];
          dp[4 * j + i] = nv[i];
        }
      }
#pragma unroll
      for (int t = 0; t < HD; ++t) {
        s = mfma32(qa[t], kf[t], s);
        dp = mfma32(da[t], vf[t], dp);
      }
      float p[16], ds[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qq = qr0 + crow(i, h);
        const bool ok = qq >= lo && qq < hi && allowed32(qq, key, W, S);
        p[i] = ok ? exp2f(s[i] - l2[i]) : 0.f;
        ds[i] = p[i] * dp[i];
      }
      // dV^T += dO^T P and dK^T += Q^T dS: lane (r, h) supplies dO / Q[qr0 + crow(t, h)][32 db + r]
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int d = 32 * db + r;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const int qq = qr0 + crow(t, h);
          const bool in = d < D && qq < L;
          const float doa = in ? dO[int64_t(qq) * a.sdo[2] + d] : 0.f;
          const float qa2 = in ? Q[int64_t(qq) * a.sq[2] + d] : 0.f;
          dv[db] = mfma32(doa, p[t], dv[db]);
          dk[db] = mfma32(qa2, ds[t], dk[db]);
        }
      }
    }
  }
  // outputs: lane (r, h) register i of tile db holds head-dim index 32 db + crow(i, h) of key ks0 + r
  if (key >= L) return;
  if (split) {
    const int64_t slot = ((int64_t(b) * a.Hkv + kvh) * a.nsp + kt) * (a.n_chunks + 1) + (chunk + 1);
    float* pk = a.partial + slot * 2 * 32 * D + r * D;
    float* pv = pk + 32 * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * db + 8 * j + 4 * h;
        if (d < D) {
          st4f(pk + d, f32x4{dk[db][4 * j], dk[db][4 * j + 1], dk[db][4 * j + 2], dk[db][4 * j + 3]});
          st4f(pv + d, f32x4{dv[db][4 * j], dv[db][4 * j + 1], dv[db][4 * j + 2], dv[db][4 * j + 3]});
        }
      }
    return;
  }
  float* dK = static_cast<float*>(a.dk) + slice_off(a.sdk, b, kvh, sq.row + key);
  float* dV = static_cast<float*>(a.dv) + slice_off(a.sdv, b, kvh, sq.row + key);
  const float sc = a.scale;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * db + 8 * j + 4 * h;
      if (d < D) {
        st4f(dK + d, f32x4{dk[db][4 * j] * sc, dk[db][4 * j + 1] * sc, dk[db][4 * j + 2] * sc, dk[db][4 * j + 3] * sc});
        st4f(dV + d, f32x4{dv[db][4 * j], dv[db][4 * j + 1], dv[db][4 * j + 2], dv[db][4 * j + 3]});
      }
    }
}

// Adds the partial sums of the split sink tiles, slot by slot in order (deterministic).  Grid
// (32 nsp, Hkv, B): one workgroup of D threads per key of a split tile.
template <int D>
__global__ __launch_bounds__(128) void fold32_kernel(const Args a) {
  const int kvh = blockIdx.y, b = blockIdx.z;
  const Seq sq = seq_of(a, b);
  const int kt = blockIdx.x / 32, r = blockIdx.x % 32, d = threadIdx.x;
  const int ks0 = 32 * kt, key = ks0 + r;
  if (key >= sq.L || d >= D) return;
  if (!(ks0 < a.S && kv32_row_end(ks0, sq.L, a.W) < sq.L && kt < a.nsp)) return;  // not split: written directly
  const int64_t slot0 = ((int64_t(b) * a.Hkv + kvh) * a.nsp + kt) * (a.n_chunks + 1);
  float sk = 0.f, sv = 0.f;
  for (int c = 0; c <= a.n_chunks; ++c) {
    const float* pk = a.partial + (slot0 + c) * 2 * 32 * D + r * D + d;
    // chunks that start past the sequence's end wrote nothing: skip them
    if (c > 0 && kv32_row_end(ks0, sq.L, a.W) + (c - 1) * a.chunk_rows >= sq.L) break;
    sk += pk[0];
    sv += pk[32 * D];
  }
  static_cast<float*>(a.dk)[slice_off(a.sdk, b, kvh, sq.row + key) + d] = sk * a.scale;
  static_cast<float*>(a.dv)[slice_off(a.sdv, b, kvh, sq.row + key) + d] = sv;
}

}  // namespace

hipError_t launch_fwd_f32(const Args& a, int D, hipStream_t s) {
  const dim3 grid((a.L + 31) / 32, a.Hq, a.B), block(64);
  switch (D) {
    case 16: hipLaunchKernelGGL(fwd32_kernel<16>, grid, block, 0, s, a); break;
    case 32: hipLaunchKernelGGL(fwd32_kernel<32>, grid, block, 0, s, a); break;
    case 64: hipLaunchKernelGGL(fwd32_kernel<64>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(fwd32_kernel<128>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_dq_f32(const Args& a, int D, hipStream_t s) {
  const dim3 grid((a.L + 31) / 32, a.Hq, a.B), block(64);
  switch (D) {
    case 16: hipLaunchKernelGGL(dq32_kernel<16>, grid, block, 0, s, a); break;
    case 32: hipLaunchKernelGGL(dq32_kernel<32>, grid, block, 0, s, a); break;
    case 64: hipLaunchKernelGGL(dq32_kernel<64>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(dq32_kernel<128>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv_f32(const Args& a, int D, hipStream_t s) {
  const dim3 grid(a.n_kblocks + a.nsp * a.n_chunks, a.Hkv, a.B), block(64);
  switch (D) {
    case 16: hipLaunchKernelGGL(dkdv32_kernel<16>, grid, block, 0, s, a); break;
    case 32: hipLaunchKernelGGL(dkdv32_kernel<32>, grid, block, 0, s, a); break;
    case 64: hipLaunchKernelGGL(dkdv32_kernel<64>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(dkdv32_kernel<128>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.nsp == 0) return e;
  const dim3 fgrid(32 * a.nsp, a.Hkv, a.B), fblock(128);
  switch (D) {
    case 16: hipLaunchKernelGGL(fold32_kernel<16>, fgrid, fblock, 0, s, a); break;
    case 32: hipLaunchKernelGGL(fold32_kernel<32>, fgrid, fblock, 0, s, a); break;
    case 64: hipLaunchKernelGGL(fold32_kernel<64>, fgrid, fblock, 0, s, a); break;
    case 128: hipLaunchKernelGGL(fold32_kernel<128>, fgrid, fblock, 0, s, a); break;
  }
  return hipGetLastError();
}

}  // namespace fa
