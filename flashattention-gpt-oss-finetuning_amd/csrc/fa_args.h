// fa_args.h - kernel argument block shared by the C ABI (fa_capi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

// Everything a kernel needs, passed by value through the kernarg segment.  Strides are in
// elements; sequence indices are int32 (validated: L < 2^28), offsets are formed in int64.
struct Args {
  // inputs
  const void* q;
  const void* k;
  const void* v;
  const void* o;     // backward: forward output
  const void* dout;  // backward: upstream gradient
  const float* lse;  // backward: forward statistic
  // outputs
  void* o_out;       // forward
  float* lse_out;    // forward
  void* dq;
  void* dk;
  void* dv;
  // backward workspace
  float* delta;      // row statistics: [B][Hq][Lp / 32][lse * log2(e) x 32, -delta x 32] fp32, Lp = L
                     // rounded up to 32 (written by the dQ kernel, read by the dK/dV kernel)
  float* partial;    // sink-key partial sums, see fa_bwd.hip
  // learned per-head sink logits (GPT-OSS): NULL, or [Hq] fp32 logits that join every row's
  // softmax denominator without a value row
  const float* sink_logits;
  float* dsink;      // backward: [Hq] fp32 gradient of the sink logits (NULL: not computed)
  float* dsink_part; // backward workspace: [B][Hq][Lp / 32] per-32-row partial sums of dsink
  int64_t sq[3], sk[3], sv[3], so[3], sdo[3], slse[3], sdq[3], sdk[3], sdv[3], so_out[3];
  int B, Hq, Hkv, L, G, Lp;
  int W, S;          // window and sink, clamped to [0, L]
  float scale;       // softmax scale as given
  float c;           // |scale| * log2(e), kept > 0: scores enter exp2 as s * c
  uint32_t qsign;    // 0x80008000 when scale < 0: flips the sign of Q in the score product
                     // (0x80808080 for e4m3 inputs)
  float oscale;      // forward with e4m3 inputs: O is multiplied by V's dequantisation factor
  // q-major kernels (forward, dQ): a workgroup is wq x wh waves, each wave 32 rows x HPW heads
  int wq, wh;
  int n_qtiles;
  // KV-major kernel (dK/dV)
  int n_kblocks;     // ceil(L / 64)
  int nsp;           // leading 64-key blocks whose sink rows are split into chunks
  int n_chunks;      // chunks of chunk_rows query rows per chunked block (0 when nsp == 0)
  int chunk_rows;
  int n_chunk_wgs;   // B * Hkv * nsp * n_chunks
  int srows;         // sink rows stored per block in the partial sums: min(S, 64)
  // sink rows in the dQ kernel (dq_sink_mode): rows past key block 0's window add the sink keys'
  // dK/dV there
  int sink_dq;       // 1 in that mode
  float* dq_sink_part;  // [n_tiles][dK, dV][srows][D] fp32: a run's sums at the slot of its first tile
  int dq_wgs;           // the dQ kernel's grid (set for the sink fold)
  // The sliding dQ kernel (fa_bwd_slide.hip), when it runs instead of bwd_dq_kernel (dq_slide = 1),
  // and the sliding forward (fa_fwd.hip fwd_slide_kernel): their workgroups ("units") take slide_ct
  // consecutive 32-row tiles of 8 query heads; a (batch, KV head, head group of 8) has slide_ncu
  // units, in that order (chunks fastest).  In dq_sink_mode dQ unit u writes slot u of
  // dq_sink_part.
  int dq_slide;
  int slide_ct;
  int slide_ncu;
  // variable-length batches: NULL, or [B + 1] device offsets of the sequences' first rows in
  // tensors of total_rows packed rows (L is then the longest sequence, batch strides are 0)
  const int* cu_seqlens;
  int total_rows;
  // Packed batches: the sliding kernels' units and the dK/dV kernel's 64-key workgroups are handed
  // out over the pieces the sequences hold (varlen_nth), so no workgroup is launched for a piece
  // past a short sequence's end.  vl_units units per (KV head, head group) and vl_kblocks key
  // blocks per KV head bound those pieces; 0: the fixed-length enumeration (B x slide_ncu units,
  // B x n_kblocks blocks).
  int vl_units;
  int vl_kblocks;
};

// Sequence b: its length and the row where it starts in the packed tensors (fixed-length
// batches: L rows from row 0 of batch b's slice).  Offsets are clamped to the tensors' rows and
// lengths to L, so malformed offsets cannot address memory outside the tensors.
struct Seq {
  int L;
  int64_t row;
};

template <typename A>
__device__ __forceinline__ Seq seq_of(const A& a, int b) {
  if (!a.cu_seqlens) return Seq{a.L, 0};
  int lo = a.cu_seqlens[b], hi = a.cu_seqlens[b + 1];
  lo = lo < 0 ? 0 : (lo > a.total_rows ? a.total_rows : lo);
  hi = hi < lo ? lo : (hi > a.total_rows ? a.total_rows : hi);
  const int n = hi - lo;
  return Seq{n < a.L ? n : a.L, lo};
}

// Packed batches: sequence b holds ceil(ceil(L_b / rows) / per) pieces of `per` blocks of `rows`
// rows, and `slots` >= their number N of workgroups enumerate them, the sequences' pieces in order
// after slots - N that have none (so that the empty ones, which exit at once, are dispatched
// first and every piece gets a place in the first round).  For the wave-uniform slot index p, sets
// b and the piece's index within its sequence and returns true, or returns false for an empty
// slot.  Wave-wide prefix sums over the sequences, 64 per round: every lane of the wave must call
// it.  (The results are made scalar so that the callers' index arithmetic stays scalar.)
template <typename A>
__device__ inline bool varlen_nth(const A& a, int p, int slots, int rows, int per, int& b, int& piece) {
  const int lane = threadIdx.x & 63;
  auto count = [&](int bb) { return bb < a.B ? ((seq_of(a, bb).L + rows - 1) / rows + per - 1) / per : 0; };
  auto prefix = [&](int n) {  // inclusive prefix sum over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(n, o);
      if (lane >= o) n += y;
    }
    return n;
  };
  int total = 0;
  for (int b0 = 0; b0 < a.B; b0 += 64) total += __builtin_amdgcn_readfirstlane(__shfl(prefix(count(b0 + lane)), 63));
  p -= slots - total;
  if (p < 0) return false;
  int base = 0;
  for (int b0 = 0; b0 < a.B; b0 += 64) {
    const int n = count(b0 + lane);
    const int x = prefix(n);
    const int tot = __builtin_amdgcn_readfirstlane(__shfl(x, 63));
    if (p < base + tot) {
      const unsigned long long m = __ballot(base + x > p);
      const int l = __builtin_amdgcn_readfirstlane(__ffsll(m) - 1);  // the first sequence whose pieces reach past p
      b = b0 + l;
      piece = __builtin_amdgcn_readfirstlane(p - base - (__shfl(x, l) - __shfl(n, l)));
      return true;
    }
    base += tot;
  }
  return false;
}

// Element offset of row `row` of (batch b, head h) of a tensor with strides s[3] (a plain array
// or one read through args_fresh()).
template <typename S3>
__device__ __forceinline__ int64_t slice_off(const S3& s, int b, int h, int64_t row) {
  return int64_t(b) * s[0] + int64_t(h) * s[1] + row * s[2];
}

#if defined(__HIP_DEVICE_COMPILE__)
// The kernel's Args in the kernarg segment (constant address space), re-read at the point of
// use.  Fields read through the by-value parameter are loaded once at kernel entry and stay in
// scalar registers for the whole kernel; the many pointers and 64-bit strides that only the
// per-tile address arithmetic needs then spill scalar registers into vector lanes inside the key
// loops.  The empty asm hides where the pointer comes from, so the loads through each call's
// result are issued after the call, where the fields are used (scalar-cache hits).
using KArgs = const __attribute__((address_space(4))) Args;
__device__ __forceinline__ KArgs& args_fresh() {
  KArgs* p = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *p;
}
#else
using KArgs = const Args;
__device__ KArgs& args_fresh();  // device code only
#endif

// Rows of a packed (variable-length) batch that belong to no sequence -- [0, cu_seqlens[0]) and
// [cu_seqlens[B], total_rows) -- are written by no attention kernel.  varlen_tail_kernel fills
// them in up to three outputs: every (row, head) of tensor i gets `cols[i]` elements of
// `elem_bytes[i]` bytes (2 or 4) set to the bit pattern `fill[i]`.  Strides are in elements.
struct TailArgs {
  const int* cu_seqlens;
  int batch, total_rows, n;
  void* ptr[3];
  int64_t head_stride[3], row_stride[3];
  int heads[3], cols[3], elem_bytes[3];
  uint32_t fill[3];
};

// Launchers (return the hipError_t of the launch; launch_bwd_dkdv also launches the sink fold).
hipError_t launch_fwd(const Args& a, int dtype, int D, int hpw, hipStream_t stream);
// e4m3 q, k, v; bf16 o; fp8_pv: P V on the fp8 MFMA as well
hipError_t launch_fwd_fp8(const Args& a, int D, int hpw, bool fp8_pv, hipStream_t stream);
hipError_t launch_bwd_dq(const Args& a, int dtype, int D, int hpw, hipStream_t stream);
// the sliding dQ kernel (D = 64, 16-bit, G a multiple of 8, 1 <= W <= 161, S <= 32)
hipError_t launch_bwd_dq_slide(const Args& a, int dtype, hipStream_t stream);
// the sliding forward (the same, W <= 129; reads slide_ct / slide_ncu)
hipError_t launch_fwd_slide(const Args& a, int dtype, hipStream_t stream);
hipError_t launch_bwd_dkdv(const Args& a, int dtype, int D, hipStream_t stream);
hipError_t launch_bwd_sink_logits(const Args& a, hipStream_t stream);  // after launch_bwd_dq
hipError_t launch_varlen_tail(const TailArgs& t, hipStream_t stream);
// float32 inputs (fa_f32.hip).  The dK/dV launch reads n_kblocks (32-key tiles), nsp (sink tiles
// that may be split), n_chunks and chunk_rows (their chunk workgroups) and launches the fold.
hipError_t launch_fwd_f32(const Args& a, int D, hipStream_t stream);
hipError_t launch_bwd_dq_f32(const Args& a, int D, hipStream_t stream);
hipError_t launch_bwd_dkdv_f32(const Args& a, int D, hipStream_t stream);

}  // namespace fa
