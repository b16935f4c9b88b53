// fa_common.h - device building blocks shared by the gfx950 attention kernels.
//
// Every kernel in this library is written around one CDNA4 matrix instruction,
// v_mfma_f32_32x32x16_{bf16,f16}: a wave64 multiplies a 32x16 A tile by a 16x32 B tile and
// accumulates a 32x32 fp32 C tile.  Lane l (r = l % 32, h = l / 32) supplies
//     A[r][8h .. 8h+7]   and   B[8h .. 8h+7][r]          (8 x 16-bit each)
// and holds
//     C[8*(i/4) + 4h + (i%4)][r]   for i = 0..15          (16 x fp32).
// (Checked on hardware by an in-bounds probe before these kernels were written.)
//
// Two consequences shape the kernels:
//  * The order of the 16 reduction indices inside one instruction is free as long as A and B
//    agree, so each kernel picks whatever index order makes its loads contiguous.
//  * A C tile holds, per lane, one column and 16 rows.  Feeding it back as the B operand of
//    the next product (after a cast to 16 bit) needs no data movement if the next product's
//    reduction index order is "rows 8j+4h..8j+4h+3 for j = 2t, 2t+1" in step t.  The matching
//    A operand is staged in LDS with the middle two quads of every 16 swapped (perm16 below),
//    so a lane reads its 8 A values with one 16-byte ds_read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_plan.h"

namespace fa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// 16-bit element types.  `Elem` selects the MFMA flavour and the fp32 -> 16-bit cast
// (round-to-nearest-even through v_cvt_pk_{bf16,f16}_f32).
struct BF16 {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // v_mfma_f32_16x16x32_bf16: lane l supplies A[l % 16][8(l/16) .. +8) and B[8(l/16) .. +8)[l % 16]
  // and holds C[4(l/16) + i][l % 16], i = 0..3 (checked on hardware by an in-bounds probe).
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  }
  static __device__ __forceinline__ float to_f32(uint16_t bits) {
    return __builtin_bit_cast(float, uint32_t(bits) << 16);
  }
  // acc + lo + hi of a packed pair (v_dot2 with ones)
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair),
                                           __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
  }
  // acc + a.lo * b.lo + a.hi * b.hi of two packed pairs (v_dot2, fp32 accumulation)
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc,
                                           false);
  }
};

struct F16 {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
  static __device__ __forceinline__ float to_f32(uint16_t bits) {
    return float(__builtin_bit_cast(_Float16, bits));
  }
  static __device__ __forceinline__ float sum2(uint32_t pair, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), __builtin_bit_cast(f16x2, 0x3c003c00u), acc,
                                  false);
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
  }
};

// FP8 (OCP e4m3) operands.
// v_mfma_scale_f32_32x32x64_f8f6f4 with unit block scales (E8M0 127 = 2^0): C += A B with A 32 x 64
// and B 64 x 32 in e4m3; lane l supplies row l % 32 of A (column l % 32 of B) and the 32 bytes
// [32 (l / 32), +32) of the K dimension, as two 16-byte halves (lo, hi); C is laid out as for
// the 32x32 bf16 form (checked on hardware by an in-bounds probe against a CPU product).
__device__ __forceinline__ f32x16 mfma_fp8(u32x4 a_lo, u32x4 a_hi, u32x4 b_lo, u32x4 b_hi, f32x16 c) {
  const i32x8 a = {int(a_lo[0]), int(a_lo[1]), int(a_lo[2]), int(a_lo[3]),
                   int(a_hi[0]), int(a_hi[1]), int(a_hi[2]), int(a_hi[3])};
  const i32x8 b = {int(b_lo[0]), int(b_lo[1]), int(b_lo[2]), int(b_lo[3]),
                   int(b_hi[0]), int(b_hi[1]), int(b_hi[2]), int(b_hi[3])};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// Sixteen e4m3 values (16 bytes) -> sixteen bf16 (two 16-byte chunks, same order), exactly
// (every finite e4m3 value is a bf16 value; v_cvt_scalef32_pk_bf16_fp8 with scale 1, checked on
// hardware over all 256 byte values).
__device__ __forceinline__ void fp8x16_to_bf16(u32x4 x, u32x4& lo, u32x4& hi) {
  uint32_t o[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    o[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[w], 1.0f, false));
    o[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x[w], 1.0f, true));
  }
  lo = u32x4{o[0], o[1], o[2], o[3]};
  hi = u32x4{o[4], o[5], o[6], o[7]};
}

// Four fp32 values -> four e4m3 bytes, in order (v_cvt_pk_fp8_f32: round to nearest even, checked
// on hardware against the OCP encoding for every finite value; |x| <= 448 assumed).
__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}
// v_permlane32_swap: lanes 32..63 of x trade values with lanes 0..31 of y (checked on hardware).
__device__ __forceinline__ void swap_halves(uint32_t& x, uint32_t& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  x = r[0];
  y = r[1];
}

// Eight fp32 C values -> one 16-byte B operand.
template <typename E>
__device__ __forceinline__ u32x4 pack8(const float* x) {
  u32x4 r;
  r[0] = E::pack2(x[0], x[1]);
  r[1] = E::pack2(x[2], x[3]);
  r[2] = E::pack2(x[4], x[5]);
  r[3] = E::pack2(x[6], x[7]);
  return r;
}

// acc + the dot product of two 16-byte vectors of 16-bit values, accumulated in fp32 (four
// v_dot2 instructions).
template <typename E>
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
#pragma unroll
  for (int w = 0; w < 4; ++w) acc = E::dot2(a[w], b[w], acc);
  return acc;
}

// Storage position of index r (0..15) inside a 16-group of a "permuted" LDS row: the middle
// two quads are swapped, so lane half h finds C rows {4h..4h+3, 8+4h..8+4h+3} at positions
// 8h..8h+7.
__device__ __forceinline__ int perm16(int r) { return (r & 3) | ((r & 4) << 1) | ((r & 8) >> 1); }
__device__ __forceinline__ int perm_pos(int idx) { return (idx & ~15) | perm16(idx & 15); }

// Output-row order of the A operand for products whose C rows are the head dim: A row m holds
// head-dim index sigma(m), so lane half h of a C tile owns head-dim indices 16h..16h+15 in
// register order i = 0..15 (contiguous, storable with two 16-byte writes).
__device__ __forceinline__ int sigma32(int m) { return ((m >> 2) & 1) * 16 + (m >> 3) * 4 + (m & 3); }

// Global loads/stores of 16 bytes.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x4 zero16() { return u32x4{0u, 0u, 0u, 0u}; }
__device__ __forceinline__ u32x4 lds16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Buffer resources: a scalar descriptor of [base, base + bytes); vector loads at byte offsets
// >= bytes return zeros, so tile edges need no branches.  (0x00020000: 32-bit data format of
// the gfx9 descriptor word 3.)
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_ld16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float buf_ldf(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
// LDS DMA (buffer_load_dwordx4 ... lds): every lane loads 16 bytes at byte offset `off` of the
// buffer, and lane l's bytes land at lds_dst + 16 l (lds_dst is wave-uniform).  Out-of-range
// offsets land zeros.  Completion is counted by vmcnt like any load; an LDS read of the data
// must wait for it explicitly: the compiler's own waits for these DMAs (before every transposed
// LDS read, which it cannot tell apart from the DMA's destination) are not placed for that.
// (Checked on hardware.)
__device__ __forceinline__ void buf_dma16(rsrc_t r, uint16_t* lds_dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds_dst), 16, off, 0, 0, 0);
}
// The same DMA issued from inline assembly, which the compiler does not see: it adds no wait for
// it before transposed LDS reads, and where it waits for an earlier load into registers
// (s_waitcnt vmcnt(n), counted from the loads it knows of) it does not wait for this one when it
// was issued after a wait it cannot see.  Only for kernels whose every wait for it is explicit.
// (M0 holds the LDS address; the s_nop covers the M0-write-to-LDS-DMA hazard.)
__device__ __forceinline__ void buf_dma16_asm(rsrc_t r, uint16_t* lds_dst, uint32_t off) {
  const uint32_t la = uint32_t(size_t((__attribute__((address_space(3))) uint16_t*)lds_dst));
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %2, %0, 0 offen lds" ::"s"(r), "{m0}"(la), "v"(off) : "memory");
}
// LDS DMA of 4 bytes per lane (buffer_load_dword ... lds): lane l's word lands at lds_dst + 4 l.
__device__ __forceinline__ void buf_dma4(rsrc_t r, uint16_t* lds_dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds_dst), 4, off, 0, 0, 0);
}
// s_waitcnt immediate (gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
// that waits until at most `vm` vector-memory loads of the wave are outstanding and every LDS
// operation has completed; exports are not waited for.
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | (((vm >> 4) & 3) << 14) | (7 << 4); }
// That wait, then the workgroup barrier.  Inline assembly, so that the compiler neither drops nor
// relaxes the wait: it does not track the LDS writes of DMA loads.
template <int VM>
__device__ __forceinline__ void wait_vm_lgkm0_barrier() {
  static_assert(VM >= 0 && VM <= 63, "vmcnt range");
  asm volatile("s_waitcnt %0\n\ts_barrier" ::"n"(waitcnt_vm_lgkm0(VM)) : "memory");
}

// The same wait without the barrier: for LDS that only the waiting wave's own DMA writes.
template <int VM>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(VM >= 0 && VM <= 63, "vmcnt range");
  asm volatile("s_waitcnt %0" ::"n"(waitcnt_vm_lgkm0(VM)) : "memory");
}

// Bytes spanned by `rows` fp32 values with stride `stride` (0 if none).
__device__ __forceinline__ uint32_t span_f32(int rows, int64_t stride) {
  return rows > 0 ? uint32_t((int64_t(rows - 1) * stride + 1) * 4) : 0u;
}
// Bytes spanned by `rows` rows of `cols` elements of `eb` bytes (16-bit by default) with row
// stride `stride` elements (0 if none).
__device__ __forceinline__ uint32_t span_bytes(int rows, int64_t stride, int cols, int eb = 2) {
  return rows > 0 ? uint32_t((int64_t(rows - 1) * stride + cols) * eb) : 0u;
}

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, output lane i, element j is
// element (i & 3) of the 8 bytes addressed by lane 4j + (i >> 2) of the group.  (Checked on
// hardware by an in-bounds probe.)  Reading 4 rows x 16 columns of a row-major LDS tile this way
// hands each lane one column and 4 consecutive rows: a transposed read with no extra LDS copy.
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 ds_read_tr16(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// ds_read_b64_tr_b8 (gfx950): within each group of 16 lanes, output lane i, byte j is byte i % 8 of
// the 8 bytes addressed by lane 2j + i / 8 of the group.  (Checked on hardware by an in-bounds
// probe.)  Reading 8 rows x 16 byte columns of a row-major LDS tile this way hands each lane one
// column and 8 consecutive rows.
typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2 ds_read_tr8(const uint16_t* p) {
  const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// A operand of v_mfma_f32_32x32x16 whose rows are head-dim indices and whose reduction index
// runs over tile rows, read from a row-major LDS tile [rows][ROW] (16-bit elements):
// lane (r = lane % 32, h = lane / 32) receives column col0 + sigma32(r) of tile rows
// {r0 + 4h + 0..3, r0 + 8 + 4h + 0..3} -- the row order of a C tile fed back as B operand.
// `ncols` columns exist; lanes whose column is >= ncols get zeros (only D = 16 has such lanes).
template <int ROW>
__device__ __forceinline__ u32x4 tr_frag(const uint16_t* tile, int r0, int col0, int ncols) {
  const int lane = threadIdx.x & 63;
  const int s = lane & 15, rh = (lane >> 4) & 1, hf = lane >> 5;
  int col = col0 + sigma32(16 * rh + 4 * (s & 3));
  if (col >= ncols) col = 0;  // any valid address; those lanes are zeroed below
  const uint16_t* p = tile + (r0 + 4 * hf + (s >> 2)) * ROW + col;
  const u32x2 lo = ds_read_tr16(p), hi = ds_read_tr16(p + 8 * ROW);
  u32x4 r = {lo[0], lo[1], hi[0], hi[1]};
  if (col0 + sigma32(lane & 31) >= ncols) r = zero16();
  return r;
}

// Swizzled [rows][D] tiles of 16-bit values in LDS (row stride D, no padding): chunk j (8
// elements, 16 bytes) of row r is stored at chunk j ^ swz(r).  With 128 bytes per LDS cycle
// (32 banks of 4 bytes) the swizzle keeps both access patterns of the kernels conflict-free:
//  * 16-byte row reads (A operands: 8 consecutive rows, one chunk each) -- swz takes distinct
//    values on any 8 rows that share a bank cycle;
//  * ds_read_b64_tr_b16 (4 consecutive rows, chunks j and j ^ 2) -- swz(r) ^ swz(r') is never 0
//    or 2 for two rows of an aligned group of 4.
// swz(r + 8) = swz(r), so a tile read at rows r and r + 8 uses one base address.
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D >= 64) return (r & 1) | ((r & 2) << 1) | ((r & 4) >> 1);
  else if constexpr (D == 32) return (r >> 1) & 3;
  else return (r >> 2) & 1;
}
// element offset of (row r, element column col) in a swizzled tile
template <int D>
__device__ __forceinline__ int swz_off(int r, int col) {
  return r * D + (((col >> 3) ^ swz<D>(r)) << 3) + (col & 7);
}

// tr_frag on a swizzled [rows][D] tile (see swz): the same operand, conflict-free.
template <int D>
__device__ __forceinline__ u32x4 tr_frag_swz(const uint16_t* tile, int r0, int col0, int ncols) {
  const int lane = threadIdx.x & 63;
  const int s = lane & 15, rh = (lane >> 4) & 1, hf = lane >> 5;
  int col = col0 + sigma32(16 * rh + 4 * (s & 3));
  if (col >= ncols) col = 0;  // any valid address; those lanes are zeroed below
  const uint16_t* p = tile + swz_off<D>(r0 + 4 * hf + (s >> 2), col);
  const u32x2 lo = ds_read_tr16(p), hi = ds_read_tr16(p + 8 * D);
  u32x4 r = {lo[0], lo[1], hi[0], hi[1]};
  if (col0 + sigma32(lane & 31) >= ncols) r = zero16();
  return r;
}

// Exchange with the lane 32 positions away (the other half of the wave).
__device__ __forceinline__ float xor32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                       int((threadIdx.x ^ 32) & 63) << 2, __builtin_bit_cast(int, x)));
}

// v_permlane32_swap v_a, v_b swaps the upper 32 lanes of v_a with the lower 32 lanes of v_b.
// Given the same value x in both, v_a ends up holding x of lane (l & 31) and v_b x of lane
// (l & 31) + 32, on every lane (checked on hardware), so max/sum of the two wave halves need no
// LDS round trip and both halves get bitwise the same result.  Written as inline asm: the
// builtin's second result is miscompiled at -O3 by the ROCm 7.2 compiler (folded into the
// first).  The s_nop covers the VALU-write -> permlane-read hazard of the operands.
__device__ __forceinline__ void halves(float x, float& lo, float& hi) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_halves(float x) {
  float lo, hi;
  halves(x, lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float sum_halves(float x) {
  float lo, hi;
  halves(x, lo, hi);
  return lo + hi;
}

// True on every lane when the predicate holds on any active lane (wave-uniform branch).
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Map a linear workgroup id to a logical tile id so that every XCD (workgroups are dispatched
// round-robin over the 8 XCDs) receives one contiguous range of logical tiles; neighbouring
// tiles share K/V rows, which then stay in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int id, int n) {
  constexpr int kXcd = 8;
  const int per = n / kXcd, rem = n % kXcd;
  const int xcd = id % kXcd, pos = id / kXcd;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + pos;
}

// Four 16-byte rows of 8 x 16-bit values -> eight 8-byte columns (4 x 16-bit), i.e. the
// 4x8 -> 8x4 transpose used to stage a [rows][d] tile as [d][rows] in LDS.
__device__ __forceinline__ void transpose4x8(const u32x4 in[4], u32x2 out[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t a = in[0][w], b = in[1][w], c = in[2][w], d = in[3][w];
    // column 2w takes the low halves, column 2w+1 the high halves
    out[2 * w][0] = (a & 0xffffu) | (b << 16);
    out[2 * w][1] = (c & 0xffffu) | (d << 16);
    out[2 * w + 1][0] = (a >> 16) | (b & 0xffff0000u);
    out[2 * w + 1][1] = (c >> 16) | (d & 0xffff0000u);
  }
}

}  // namespace fa
