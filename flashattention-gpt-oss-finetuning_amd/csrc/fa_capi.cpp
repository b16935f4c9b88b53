// fa_capi.cpp - the C ABI declared in include/fa_gfx950.h: host-side validation, workspace
// sizing, launch-shape selection and dispatch to the gfx950 kernels.
//
// Validation mirrors the reference's checks (flash_attention_gpt_oss.py:343-354:
// causal only, shape agreement, D <= 128, Hq % Hkv == 0; benchmark_backward_speed.py:476-484)
// plus what the kernels assume (16-byte aligned rows, D in {16, 32, 64, 128}).  Nothing in
// fa_check_* touches HIP, so the checks run on machines without a GPU.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/fa_gfx950.h"
#include "fa_args.h"
#include "fa_plan.h"

namespace {

constexpr int64_t kMaxSeq = int64_t(1) << 28;
constexpr int kChunkRows = 64;  // query rows per sink-chunk workgroup of the dK/dV kernel

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// strides in elements of `elem_bytes` bytes: non-negative and whole 16-byte multiples
bool strides_ok(const int64_t s[3], int elem_bytes = 2) {
  const int64_t m = 16 / elem_bytes - 1;
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] & m) != 0) return false;
  return true;
}

bool lse_strides_ok(const int64_t s[3]) { return s[0] >= 0 && s[1] >= 0 && s[2] >= 0; }

bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// The kernels address one (batch, head) slice of a tensor with 32-bit byte offsets: its L rows
// must span fewer than 2^31 bytes.
bool slice_fits(const int64_t s[3], int L, int D, int elem_bytes) {
  return (int64_t(L - 1) * s[2] + D) * elem_bytes < (int64_t(1) << 31);
}

// bytes per element of q/k/v/o/dout/dq/dk/dv for a 16-bit or float32 call
int elem_bytes(int32_t dtype) { return dtype == FA_DTYPE_F32 ? 4 : 2; }

int check_common(int32_t B, int32_t Hq, int32_t Hkv, int32_t L, int32_t D, int32_t W, int32_t S,
                 float scale, int32_t dtype) {
  if (B < 1 || Hq < 1 || Hkv < 1 || L < 1) return FA_ERR_SHAPE;
  if (Hq % Hkv != 0) return FA_ERR_SHAPE;
  if (D != 16 && D != 32 && D != 64 && D != 128) return FA_ERR_HEAD_DIM;
  if (dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F16 && dtype != FA_DTYPE_F32) return FA_ERR_DTYPE;
  if (W < 1 && S < 1) return FA_ERR_MASK;
  if (!std::isfinite(scale)) return FA_ERR_SCALE;
  if (int64_t(L) > kMaxSeq) return FA_ERR_OVERFLOW;
  // grid sizes of the launches must fit 32 bits
  if (int64_t(B) * Hq * ((int64_t(L) + 31) / 32) > (int64_t(1) << 31)) return FA_ERR_OVERFLOW;
  return FA_OK;
}

// Workgroup shape of the query-major kernels: wq waves along the sequence x wh waves along the
// heads, each wave 32 rows x hpw heads (hpw <= hmax); hpw * wh heads must divide the group size
// so that a workgroup never straddles two KV heads.  The forward shares each K/V fragment
// between two heads of a wave for D <= 64; the dQ kernel keeps one head per wave, which leaves
// it two waves per SIMD (measured faster at D = 64).
void choose_qmajor(int G, int hmax, int* hpw, int* wh, int* wq) {
  for (int h = hmax; h >= 1; --h)
    for (int w = 4; w >= 1; w /= 2)
      if (G % (h * w) == 0) {
        *hpw = h;
        *wh = w;
        *wq = 4 / w;
        return;
      }
  *hpw = 1;
  *wh = 1;
  *wq = 4;
}

struct SinkPlan {
  int nsp, n_chunks, srows;  // chunked blocks, chunks per block, stored sink rows per block
  int dq;                    // sink rows past block 0's window go through the dQ kernel
};

SinkPlan sink_plan(int L, int W, int S) {
  // clamp as the kernels do
  W = W < 0 ? 0 : (W > L ? L : W);
  S = S < 0 ? 0 : (S > L ? L : S);
  SinkPlan p{0, 0, 0, 0};
  p.nsp = fa::kv_sink_blocks(L, W, S);
  p.dq = fa::dq_sink_mode(L, W, S) ? 1 : 0;
  p.n_chunks = p.dq ? 0 : fa::kv_n_chunks(L, W, S, kChunkRows);
  p.srows = S < fa::kKvKeys ? S : fa::kKvKeys;
  return p;
}

// Tiles of the dQ kernel: row tiles of 32 * wq rows times head groups of wh heads (one query
// head per wave).
int64_t dq_tiles(int B, int Hq, int Hkv, int L) {
  int hpw, wh, wq;
  choose_qmajor(Hq / Hkv, 1, &hpw, &wh, &wq);
  const int64_t n_qtiles = (int64_t(L) + 32 * wq - 1) / (32 * wq);
  return n_qtiles * B * (Hq / wh);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// per-32-row-block partial sums of the learned sink logits' gradient: [B][Hq][Lp / 32] fp32
size_t dsink_part_bytes(int B, int Hq, int L) { return align256(size_t(B) * Hq * ((size_t(L) + 31) / 32) * sizeof(float)); }

// row statistics of the backward: [B][Hq][Lp / 32][lse * log2(e) x 32, -delta x 32] fp32
size_t delta_bytes(int B, int Hq, int L) {
  const size_t Lp = (size_t(L) + 31) / 32 * 32;
  return align256(size_t(B) * Hq * Lp * 2 * sizeof(float));
}

// fp32 partial sums of the sink rows: [B * Hkv][nsp][n_chunks + 1 slots][dK, dV][srows][D]
size_t partial_bytes(int B, int Hkv, int D, const SinkPlan& sp) {
  return align256(size_t(B) * Hkv * sp.nsp * (sp.n_chunks + 1) * 2 * sp.srows * D * sizeof(float));
}

// dq_sink_mode: the dQ kernel's flushed sink partials, [n_tiles][dK, dV][srows][D] fp32 (a slot
// per tile; a run of tiles writes the slot of its first tile)
size_t dq_sink_slot_bytes(int B, int Hq, int Hkv, int L, int D, const SinkPlan& sp) {
  return sp.dq ? align256(size_t(dq_tiles(B, Hq, Hkv, L)) * 2 * sp.srows * D * sizeof(float)) : 0;
}

// float32 backward: 32-key tiles; the tiles holding sink keys whose rows extend past their window
// (kv32_row_end in fa_f32.hip: min(L, 32 kt + 31 + max(W, 1))) split those rows into chunk
// workgroups of kF32ChunkRows rows, with fp32 partials [B * Hkv][nsp][n_chunks + 1][dK, dV][32][D].
constexpr int kF32ChunkRows = 256;
struct F32Plan {
  int n_kt, nsp, n_chunks;
};
F32Plan f32_plan(int L, int W, int S) {
  W = W < 0 ? 0 : (W > L ? L : W);
  S = S < 0 ? 0 : (S > L ? L : S);
  F32Plan p;
  p.n_kt = (L + 31) / 32;
  const int row_end0 = fa::imin(L, 31 + fa::imax(W, 1));  // tile 0's window rows end first
  p.n_chunks = (S > 0 && row_end0 < L) ? (L - row_end0 + kF32ChunkRows - 1) / kF32ChunkRows : 0;
  p.nsp = p.n_chunks > 0 ? (S + 31) / 32 : 0;
  return p;
}
size_t f32_partial_bytes(int B, int Hkv, int D, const F32Plan& fp) {
  return align256(size_t(B) * Hkv * fp.nsp * (fp.n_chunks + 1) * 2 * 32 * D * sizeof(float));
}
// The workspace after the row statistics and the learned-sink partials: the sink-key partials
// and dQ-kernel slots of the 16-bit backward, or the float32 backward's partials (whichever is
// larger, so one size serves every dtype).
size_t partial_region_bytes(int B, int Hq, int Hkv, int L, int D, int W, int S) {
  const SinkPlan sp = sink_plan(L, W, S);
  const size_t b16 = partial_bytes(B, Hkv, D, sp) + dq_sink_slot_bytes(B, Hq, Hkv, L, D, sp);
  const size_t b32 = f32_partial_bytes(B, Hkv, D, f32_plan(L, W, S));
  return b16 > b32 ? b16 : b32;
}

void copy3(int64_t dst[3], const int64_t src[3]) {
  for (int i = 0; i < 3; ++i) dst[i] = src[i];
}

// Compute units of the current device (256 on MI355X; 256 if the query fails).
int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n < 1)
    n = 256;
  return n;
}

// Tiles per unit (slide_ct) of the sliding kernels, for `slots` resident units.  A fixed-length
// batch spreads its B Hkv (G / 8) n_qt tiles evenly over the slots.  A packed batch holds at most
// T = ceil(total_rows / 32) + B tiles with rows (each sequence adds at most one partial tile),
// however long its longest sequence (which sets n_qt); units past a short sequence's end exit at
// once.  Its units cut every sequence separately, so a (KV head, head group of 8) needs about
// T / ct + B / 2 units (half a unit lost per sequence on average), and ct is raised until those
// fit the slots: units that spill into a second round would double the kernel's time.
int slide_units_ct(const fa::Args& a, int64_t slots) {
  const int64_t n_qt = (int64_t(a.L) + 31) / 32;
  const int64_t hg = int64_t(a.Hkv) * (a.G / 8);
  int64_t tiles = int64_t(a.B) * n_qt;
  if (a.cu_seqlens) tiles = std::min(tiles, (int64_t(a.total_rows) + 31) / 32 + a.B);
  int64_t ct = (hg * tiles + slots - 1) / slots;
  if (a.cu_seqlens) {
    const int64_t per_group = slots / hg - a.B / 2;
    if (per_group >= 1) ct = std::max(ct, (tiles + per_group - 1) / per_group);
  }
  return int(std::max<int64_t>(ct, 1));
}

// Packed batches, the sliding kernels: units per (KV head, head group) that the sequences' rows can
// fill -- sequence b needs ceil(ceil(L_b / 32) / ct) <= L_b / (32 ct) + 1 units, so at most
// ceil(total_rows / (32 ct)) + B in all -- when fewer than B x slide_ncu (see fa::Args); 0 for a
// fixed-length batch.
int vl_units(const fa::Args& a) {
  if (!a.cu_seqlens) return 0;
  const int64_t rows_ct = 32 * int64_t(a.slide_ct);
  const int64_t bound = (int64_t(a.total_rows) + rows_ct - 1) / rows_ct + a.B;
  return bound < int64_t(a.B) * a.slide_ncu ? int(bound) : 0;
}

// The sliding dQ kernel (fa_bwd_slide.hip) serves D = 64 16-bit backwards whose KV groups hold a
// multiple of 8 query heads, with a window of 1..161 keys (at most 6 key halves of 32 in LDS) and
// at most 32 sink keys (one sink half).  Its workgroups take slide_ct consecutive 32-row tiles,
// sized so that the units with rows about fill the device once.  (Any slide_ct >= 1 fits the
// workspace: the units, B Hkv (G / 8) slide_ncu, never exceed half of bwd_dq_kernel's tiles, for
// which the dQ sink slots are sized.)
void plan_slide(fa::Args& a, int D) {
  if (D != 64 || a.G % 8 != 0 || a.W < 1 || a.W > fa::kSlideMaxW || a.S > 32 || a.L < 1) return;
  const int64_t n_qt = (int64_t(a.L) + 31) / 32;
  const int64_t ct = slide_units_ct(a, device_cus());
  a.dq_slide = 1;
  a.slide_ct = int(ct);
  a.slide_ncu = int((n_qt + ct - 1) / ct);
  a.vl_units = vl_units(a);
}

// The sliding forward (fa_fwd.hip fwd_slide_kernel): the same shapes with W <= 129; two
// workgroups per CU.  Returns whether it applies (then slide_ct / slide_ncu are set).
bool plan_fwd_slide(fa::Args& a, int D, int dtype) {
  if (dtype == FA_DTYPE_F32 || D != 64 || a.G % 8 != 0 || a.W < 1 || a.W > fa::kFwdSlideMaxW || a.S > 32 ||
      a.L < 1)
    return false;
  const int64_t n_qt = (int64_t(a.L) + 31) / 32;
  const int64_t ct = slide_units_ct(a, 2 * int64_t(device_cus()));
  a.slide_ct = int(ct);
  a.slide_ncu = int((n_qt + ct - 1) / ct);
  a.vl_units = vl_units(a);
  return true;
}

// Packed batches, the dK/dV kernel: key blocks per KV head that the sequences' keys can fill
// (each sequence adds at most one partial block), when fewer than B x n_kblocks (see fa::Args).
int vl_kblocks(const fa::Args& a) {
  if (!a.cu_seqlens) return 0;
  const int64_t bound = (int64_t(a.total_rows) + fa::kKvKeys - 1) / fa::kKvKeys + a.B;
  return bound < int64_t(a.B) * a.n_kblocks ? int(bound) : 0;
}

fa::Args base_args(int32_t B, int32_t Hq, int32_t Hkv, int32_t L, int32_t D, int32_t W, int32_t S,
                   float scale) {
  fa::Args a;
  std::memset(&a, 0, sizeof(a));
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.L = L;
  a.G = Hq / Hkv;
  a.Lp = (L + 31) / 32 * 32;
  a.W = W < 0 ? 0 : (W > L ? L : W);
  a.S = S < 0 ? 0 : (S > L ? L : S);
  a.scale = scale;
  float c = std::fabs(scale) * 1.4426950408889634f;
  // A zero scale gives the uniform softmax; a tiny positive factor keeps -inf * c well defined
  // and changes no fp32 result.
  if (c < 1e-30f) c = 1e-30f;
  a.c = c;
  a.qsign = scale < 0.f ? 0x80008000u : 0u;
  (void)D;
  return a;
}

}  // namespace

extern "C" {

int fa_check_fwd(const fa_fwd_params* p) {
  if (!p) return FA_ERR_NULL;
  if (!p->q || !p->k || !p->v || !p->o || !p->lse) return FA_ERR_NULL;
  const int rc = check_common(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim, p->window,
                              p->sink, p->softmax_scale, p->dtype);
  if (rc != FA_OK) return rc;
  if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o) || !aligned4(p->lse))
    return FA_ERR_ALIGN;
  const int eb = elem_bytes(p->dtype);
  if (!strides_ok(p->q_stride, eb) || !strides_ok(p->k_stride, eb) || !strides_ok(p->v_stride, eb) ||
      !strides_ok(p->o_stride, eb) || !lse_strides_ok(p->lse_stride))
    return FA_ERR_ALIGN;
  // q, k and v are staged through buffer resources with 32-bit byte offsets inside one
  // (batch, head) slice; o and lse are written through 64-bit addresses
  const int L = p->seqlen, D = p->head_dim;
  if (!slice_fits(p->q_stride, L, D, eb) || !slice_fits(p->k_stride, L, D, eb) || !slice_fits(p->v_stride, L, D, eb))
    return FA_ERR_OVERFLOW;
  return FA_OK;
}

int fa_check_bwd(const fa_bwd_params* p) {
  if (!p) return FA_ERR_NULL;
  if (!p->q || !p->k || !p->v || !p->o || !p->dout || !p->lse || !p->dq || !p->dk || !p->dv)
    return FA_ERR_NULL;
  const int rc = check_common(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim, p->window,
                              p->sink, p->softmax_scale, p->dtype);
  if (rc != FA_OK) return rc;
  const void* ptrs[] = {p->q, p->k, p->v, p->o, p->dout, p->dq, p->dk, p->dv};
  for (const void* x : ptrs)
    if (!aligned16(x)) return FA_ERR_ALIGN;
  if (!aligned4(p->lse)) return FA_ERR_ALIGN;
  const int eb = elem_bytes(p->dtype);
  if (!strides_ok(p->q_stride, eb) || !strides_ok(p->k_stride, eb) || !strides_ok(p->v_stride, eb) ||
      !strides_ok(p->o_stride, eb) || !strides_ok(p->do_stride, eb) || !lse_strides_ok(p->lse_stride) ||
      !strides_ok(p->dq_stride, eb) || !strides_ok(p->dk_stride, eb) || !strides_ok(p->dv_stride, eb))
    return FA_ERR_ALIGN;
  // every input is read through buffer resources with 32-bit byte offsets inside one
  // (batch, head) slice; dq, dk and dv are written through 64-bit addresses
  const int L = p->seqlen, D = p->head_dim;
  if (!slice_fits(p->q_stride, L, D, eb) || !slice_fits(p->do_stride, L, D, eb) || !slice_fits(p->o_stride, L, D, eb) ||
      !slice_fits(p->lse_stride, L, 1, 4) || !slice_fits(p->k_stride, L, D, eb) || !slice_fits(p->v_stride, L, D, eb))
    return FA_ERR_OVERFLOW;
  return FA_OK;
}

}  // extern "C"

namespace {

// Variable-length batches: the sequences' rows are packed, so the batch strides are unused.
int check_varlen(const int32_t* cu_seqlens, int32_t total_rows) {
  if (!cu_seqlens) return FA_ERR_NULL;
  if (!aligned4(cu_seqlens)) return FA_ERR_ALIGN;
  if (total_rows < 0) return FA_ERR_SHAPE;
  return FA_OK;
}

// Adds tensor (ptr, strides s = batch/head/row, heads, cols, element bytes, fill bits) to the
// outputs whose uncovered packed rows varlen_tail_kernel fills.
void tail_add(fa::TailArgs* t, void* ptr, const int64_t s[3], int heads, int cols, int eb, uint32_t fill) {
  const int i = t->n++;
  t->ptr[i] = ptr;
  t->head_stride[i] = s[1];
  t->row_stride[i] = s[2];
  t->heads[i] = heads;
  t->cols[i] = cols;
  t->elem_bytes[i] = eb;
  t->fill[i] = fill;
}

fa::TailArgs tail_args(const int32_t* cu_seqlens, int32_t batch, int32_t total_rows) {
  fa::TailArgs t;
  std::memset(&t, 0, sizeof(t));
  t.cu_seqlens = cu_seqlens;
  t.batch = batch;
  t.total_rows = total_rows;
  return t;
}

void set_varlen(fa::Args* a, const int32_t* cu_seqlens, int32_t total_rows) {
  a->cu_seqlens = cu_seqlens;
  a->total_rows = total_rows;
  for (int64_t* st : {a->sq, a->sk, a->sv, a->so, a->sdo, a->slse, a->sdq, a->sdk, a->sdv, a->so_out}) st[0] = 0;
}

int run_fwd(const fa_fwd_params* p, const float* sinks, void* stream, const int32_t* cu_seqlens = nullptr,
            int32_t total_rows = 0) {
  fa::Args a = base_args(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim, p->window, p->sink,
                         p->softmax_scale);
  a.q = p->q;
  a.k = p->k;
  a.v = p->v;
  a.o_out = p->o;
  a.lse_out = p->lse;
  a.sink_logits = sinks;
  copy3(a.sq, p->q_stride);
  copy3(a.sk, p->k_stride);
  copy3(a.sv, p->v_stride);
  copy3(a.so_out, p->o_stride);
  copy3(a.slse, p->lse_stride);
  if (cu_seqlens) set_varlen(&a, cu_seqlens, total_rows);
  if (p->dtype == FA_DTYPE_F32)
    return fa::launch_fwd_f32(a, p->head_dim, static_cast<hipStream_t>(stream)) == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
  if (plan_fwd_slide(a, p->head_dim, p->dtype))
    return fa::launch_fwd_slide(a, p->dtype, static_cast<hipStream_t>(stream)) == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
  int hpw, wh, wq;
  choose_qmajor(a.G, p->head_dim <= 64 ? 2 : 1, &hpw, &wh, &wq);
  a.wh = wh;
  a.wq = wq;
  a.n_qtiles = (a.L + 32 * wq - 1) / (32 * wq);
  const hipError_t e = fa::launch_fwd(a, p->dtype, p->head_dim, hpw, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

// fa_fwd_fp8: e4m3 q, k, v (1-byte elements), bf16 o, D in {64, 128}, finite dequantisation factors.
int check_fwd_fp8(const fa_fwd_params* p, float qd, float kd, float vd) {
  if (!p) return FA_ERR_NULL;
  if (!p->q || !p->k || !p->v || !p->o || !p->lse) return FA_ERR_NULL;
  if (p->dtype != FA_DTYPE_FP8_E4M3) return FA_ERR_DTYPE;
  const int rc = check_common(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim, p->window, p->sink,
                              p->softmax_scale, FA_DTYPE_BF16);
  if (rc != FA_OK) return rc;
  if (p->head_dim != 64 && p->head_dim != 128) return FA_ERR_HEAD_DIM;
  if (!std::isfinite(qd) || !std::isfinite(kd) || !std::isfinite(vd) || !std::isfinite(p->softmax_scale * qd * kd))
    return FA_ERR_SCALE;
  if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o) || !aligned4(p->lse))
    return FA_ERR_ALIGN;
  if (!strides_ok(p->q_stride, 1) || !strides_ok(p->k_stride, 1) || !strides_ok(p->v_stride, 1) ||
      !strides_ok(p->o_stride) || !lse_strides_ok(p->lse_stride))
    return FA_ERR_ALIGN;
  const int L = p->seqlen, D = p->head_dim;
  if (!slice_fits(p->q_stride, L, D, 1) || !slice_fits(p->k_stride, L, D, 1) || !slice_fits(p->v_stride, L, D, 1))
    return FA_ERR_OVERFLOW;
  return FA_OK;
}

// The scores are (q_descale k_descale scale) * (q . k) over the stored e4m3 values; O is scaled
// by v_descale in the kernel's epilogue.
int run_fwd_fp8(const fa_fwd_params* p, float qd, float kd, float vd, const float* sinks, bool fp8_pv,
                void* stream) {
  const float scale = p->softmax_scale * qd * kd;
  fa::Args a = base_args(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim, p->window, p->sink, scale);
  a.qsign = scale < 0.f ? 0x80808080u : 0u;
  a.oscale = vd;
  a.q = p->q;
  a.k = p->k;
  a.v = p->v;
  a.o_out = p->o;
  a.lse_out = p->lse;
  a.sink_logits = sinks;
  copy3(a.sq, p->q_stride);
  copy3(a.sk, p->k_stride);
  copy3(a.sv, p->v_stride);
  copy3(a.so_out, p->o_stride);
  copy3(a.slse, p->lse_stride);
  int hpw, wh, wq;
  choose_qmajor(a.G, p->head_dim == 64 ? 2 : 1, &hpw, &wh, &wq);
  a.wh = wh;
  a.wq = wq;
  a.n_qtiles = (a.L + 32 * wq - 1) / (32 * wq);
  const hipError_t e = fa::launch_fwd_fp8(a, p->head_dim, hpw, fp8_pv, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int fa_fwd(const fa_fwd_params* p, void* stream) {
  const int rc = fa_check_fwd(p);
  return rc != FA_OK ? rc : run_fwd(p, nullptr, stream);
}

int fa_fwd_varlen(const fa_fwd_params* p, const int32_t* cu_seqlens, int32_t total_rows, const float* sinks,
                  void* stream) {
  int rc = fa_check_fwd(p);
  if (rc == FA_OK) rc = check_varlen(cu_seqlens, total_rows);
  if (rc != FA_OK) return rc;
  if (sinks && !aligned4(sinks)) return FA_ERR_ALIGN;
  rc = run_fwd(p, sinks, stream, cu_seqlens, total_rows);
  if (rc != FA_OK) return rc;
  // rows outside every sequence: o = 0, lse = -inf (an empty row)
  fa::TailArgs t = tail_args(cu_seqlens, p->batch, total_rows);
  tail_add(&t, p->o, p->o_stride, p->heads_q, p->head_dim, elem_bytes(p->dtype), 0u);
  tail_add(&t, p->lse, p->lse_stride, p->heads_q, 1, 4, 0xff800000u);
  return fa::launch_varlen_tail(t, static_cast<hipStream_t>(stream)) == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

int fa_fwd_fp8(const fa_fwd_params* p, float q_descale, float k_descale, float v_descale, const float* sinks,
               void* stream) {
  const int rc = check_fwd_fp8(p, q_descale, k_descale, v_descale);
  if (rc != FA_OK) return rc;
  if (sinks && !aligned4(sinks)) return FA_ERR_ALIGN;
  return run_fwd_fp8(p, q_descale, k_descale, v_descale, sinks, false, stream);
}

int fa_fwd_fp8_pv(const fa_fwd_params* p, float q_descale, float k_descale, float v_descale, const float* sinks,
                  void* stream) {
  const int rc = check_fwd_fp8(p, q_descale, k_descale, v_descale);
  if (rc != FA_OK) return rc;
  if (sinks && !aligned4(sinks)) return FA_ERR_ALIGN;
  return run_fwd_fp8(p, q_descale, k_descale, v_descale, sinks, true, stream);
}

int fa_fwd_sinks(const fa_fwd_params* p, const float* sinks, void* stream) {
  const int rc = fa_check_fwd(p);
  if (rc != FA_OK) return rc;
  if (!sinks) return FA_ERR_NULL;
  if (!aligned4(sinks)) return FA_ERR_ALIGN;
  return run_fwd(p, sinks, stream);
}

size_t fa_bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t seqlen,
                              int32_t head_dim, int32_t window, int32_t sink) {
  if (check_common(batch, heads_q, heads_kv, seqlen, head_dim, window, sink, 1.f, FA_DTYPE_BF16) != FA_OK)
    return 0;
  return delta_bytes(batch, heads_q, seqlen) + dsink_part_bytes(batch, heads_q, seqlen) +
         partial_region_bytes(batch, heads_q, heads_kv, seqlen, head_dim, window, sink);
}

}  // extern "C"

namespace {

// Validates a backward call and fills the kernel arguments; returns FA_OK or an fa_status.
int prepare_bwd(const fa_bwd_params* p, void* workspace, size_t workspace_bytes, fa::Args* out, int* hpw) {
  const int rc = fa_check_bwd(p);
  if (rc != FA_OK) return rc;
  const size_t need = fa_bwd_workspace_bytes(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim,
                                             p->window, p->sink);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return FA_ERR_WORKSPACE;
  fa::Args a = base_args(p->batch, p->heads_q, p->heads_kv, p->seqlen, p->head_dim, p->window, p->sink,
                         p->softmax_scale);
  a.q = p->q;
  a.k = p->k;
  a.v = p->v;
  a.o = p->o;
  a.dout = p->dout;
  a.lse = p->lse;
  a.dq = p->dq;
  a.dk = p->dk;
  a.dv = p->dv;
  copy3(a.sq, p->q_stride);
  copy3(a.sk, p->k_stride);
  copy3(a.sv, p->v_stride);
  copy3(a.so, p->o_stride);
  copy3(a.sdo, p->do_stride);
  copy3(a.slse, p->lse_stride);
  copy3(a.sdq, p->dq_stride);
  copy3(a.sdk, p->dk_stride);
  copy3(a.sdv, p->dv_stride);
  a.delta = static_cast<float*>(workspace);

  int wh, wq;
  choose_qmajor(a.G, 1, hpw, &wh, &wq);
  a.wh = wh;
  a.wq = wq;
  a.n_qtiles = (a.L + 32 * wq - 1) / (32 * wq);

  // workspace: row statistics | learned-sink partials | partial region (see partial_region_bytes)
  char* ws = static_cast<char*>(workspace);
  const size_t off_dsink = delta_bytes(a.B, a.Hq, a.L);
  a.dsink_part = reinterpret_cast<float*>(ws + off_dsink);
  a.partial = reinterpret_cast<float*>(ws + off_dsink + dsink_part_bytes(a.B, a.Hq, a.L));
  if (p->dtype == FA_DTYPE_F32) {
    const F32Plan fp = f32_plan(a.L, p->window, p->sink);
    a.n_kblocks = fp.n_kt;
    a.nsp = fp.nsp;
    a.n_chunks = fp.n_chunks;
    a.chunk_rows = kF32ChunkRows;
    *out = a;
    return FA_OK;
  }
  const SinkPlan sp = sink_plan(a.L, p->window, p->sink);
  a.sink_dq = sp.dq;
  if (sp.dq) a.dq_sink_part = a.partial + partial_bytes(a.B, a.Hkv, p->head_dim, sp) / sizeof(float);
  a.n_kblocks = (a.L + fa::kKvKeys - 1) / fa::kKvKeys;
  a.nsp = sp.nsp;
  a.n_chunks = sp.n_chunks;
  a.chunk_rows = kChunkRows;
  a.srows = sp.srows;
  a.n_chunk_wgs = a.B * a.Hkv * a.nsp * a.n_chunks;
  plan_slide(a, p->head_dim);
  *out = a;
  return FA_OK;
}

int run_dq(const fa::Args& a, const fa_bwd_params* p, int hpw, hipStream_t s) {
  const hipError_t e = p->dtype == FA_DTYPE_F32 ? fa::launch_bwd_dq_f32(a, p->head_dim, s)
                       : a.dq_slide         ? fa::launch_bwd_dq_slide(a, p->dtype, s)
                                            : fa::launch_bwd_dq(a, p->dtype, p->head_dim, hpw, s);
  return e == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

int run_dkdv(const fa::Args& a, const fa_bwd_params* p, hipStream_t s) {
  const hipError_t e = p->dtype == FA_DTYPE_F32 ? fa::launch_bwd_dkdv_f32(a, p->head_dim, s)
                                                : fa::launch_bwd_dkdv(a, p->dtype, p->head_dim, s);
  return e == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int fa_bwd(const fa_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  fa::Args a;
  int hpw = 1;
  const int rc = prepare_bwd(p, workspace, workspace_bytes, &a, &hpw);
  if (rc != FA_OK) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int r1 = run_dq(a, p, hpw, s);
  return r1 != FA_OK ? r1 : run_dkdv(a, p, s);
}

int fa_bwd_sinks(const fa_bwd_params* p, const float* sinks, float* dsinks, void* workspace, size_t workspace_bytes,
                 void* stream) {
  fa::Args a;
  int hpw = 1;
  const int rc = prepare_bwd(p, workspace, workspace_bytes, &a, &hpw);
  if (rc != FA_OK) return rc;
  if (!sinks || !dsinks) return FA_ERR_NULL;
  if (!aligned4(sinks) || !aligned4(dsinks)) return FA_ERR_ALIGN;
  a.sink_logits = sinks;
  a.dsink = dsinks;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int r = run_dq(a, p, hpw, s);
  if (r == FA_OK) r = fa::launch_bwd_sink_logits(a, s) == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
  return r != FA_OK ? r : run_dkdv(a, p, s);
}

int fa_bwd_varlen(const fa_bwd_params* p, const int32_t* cu_seqlens, int32_t total_rows, const float* sinks,
                  float* dsinks, void* workspace, size_t workspace_bytes, void* stream) {
  fa::Args a;
  int hpw = 1;
  int rc = prepare_bwd(p, workspace, workspace_bytes, &a, &hpw);
  if (rc == FA_OK) rc = check_varlen(cu_seqlens, total_rows);
  if (rc != FA_OK) return rc;
  if (!sinks != !dsinks) return FA_ERR_NULL;
  if ((sinks && !aligned4(sinks)) || (dsinks && !aligned4(dsinks))) return FA_ERR_ALIGN;
  set_varlen(&a, cu_seqlens, total_rows);
  if (a.dq_slide) plan_slide(a, p->head_dim);  // size the units by the rows the batch holds
  if (p->dtype != FA_DTYPE_F32) a.vl_kblocks = vl_kblocks(a);
  a.sink_logits = sinks;
  a.dsink = dsinks;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int r = run_dq(a, p, hpw, s);
  if (r == FA_OK && sinks) r = fa::launch_bwd_sink_logits(a, s) == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
  if (r == FA_OK) r = run_dkdv(a, p, s);
  if (r != FA_OK) return r;
  // rows outside every sequence have zero gradients
  fa::TailArgs t = tail_args(cu_seqlens, p->batch, total_rows);
  const int eb = elem_bytes(p->dtype);
  tail_add(&t, p->dq, p->dq_stride, p->heads_q, p->head_dim, eb, 0u);
  tail_add(&t, p->dk, p->dk_stride, p->heads_kv, p->head_dim, eb, 0u);
  tail_add(&t, p->dv, p->dv_stride, p->heads_kv, p->head_dim, eb, 0u);
  return fa::launch_varlen_tail(t, s) == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

int fa_bwd_dq(const fa_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  fa::Args a;
  int hpw = 1;
  const int rc = prepare_bwd(p, workspace, workspace_bytes, &a, &hpw);
  return rc != FA_OK ? rc : run_dq(a, p, hpw, static_cast<hipStream_t>(stream));
}

int fa_bwd_dkdv(const fa_bwd_params* p, void* workspace, size_t workspace_bytes, void* stream) {
  fa::Args a;
  int hpw = 1;
  const int rc = prepare_bwd(p, workspace, workspace_bytes, &a, &hpw);
  return rc != FA_OK ? rc : run_dkdv(a, p, static_cast<hipStream_t>(stream));
}

const char* fa_strerror(int status) {
  switch (status) {
    case FA_OK: return "ok";
    case FA_ERR_NULL: return "a required pointer is NULL";
    case FA_ERR_SHAPE: return "invalid shape: batch, heads and seqlen must be >= 1 and heads_q % heads_kv == 0";
    case FA_ERR_HEAD_DIM: return "head_dim must be one of 16, 32, 64, 128 (64 or 128 for fa_fwd_fp8*)";
    case FA_ERR_DTYPE: return "dtype must be FA_DTYPE_BF16, FA_DTYPE_F16 or FA_DTYPE_F32 (FA_DTYPE_FP8_E4M3 for fa_fwd_fp8*)";
    case FA_ERR_ALIGN: return "tensors must be 16-byte aligned with non-negative strides that are multiples of 16 bytes (lse: 4-byte aligned, non-negative strides)";
    case FA_ERR_MASK: return "window < 1 and sink < 1 leave every query row fully masked";
    case FA_ERR_WORKSPACE: return "workspace is NULL, not 256-byte aligned or smaller than fa_bwd_workspace_bytes()";
    case FA_ERR_LAUNCH: return "HIP kernel launch failed";
    case FA_ERR_OVERFLOW: return "problem size exceeds the kernels' index range";
    case FA_ERR_SCALE: return "softmax_scale (and the fp8 dequantisation factors) must be finite";
    case FA_ERR_SCRATCH: return "the problem needs more backward workspace than the library's scratch buffer (FA_SCRATCH_BYTES) holds; use fa_bwd with a workspace";
  }
  return "unknown fa_status";
}

int fa_version(void) { return FA_GFX950_VERSION; }

}  // extern "C"
