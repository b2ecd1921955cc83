// torque_hip.hip -- MI355X (gfx950) kernels and C ABI for the packed rotated
// KV-cache decode path.  Declarations and the reference interfaces each entry
// point replaces are in include/torque_hip.h.
//
// Kernels
//   fwht_kernel          structured Hadamard rotation, one wavefront per row
//   append_kernel        rotate -> quantize -> bit-pack (or dequantize), one
//                        wavefront per (row, stream), packed words written in
//                        place into the [L, Hkv, capacity, W] slab
//   unpack_kernel        packed slab -> dense float32 centroid values
//   decode_kernel<Fmt>   split-K decode attention: each workgroup owns one
//                        (layer, KV head, query-head group) and one split of
//                        the sequence (row blocks dealt out cyclically) and
//                        writes its partial (max, sum, accumulator); with a
//                        single split it finishes the rows itself.  Fmt
//                        selects packed 2/3/4-bit or dense fp16/fp32 rows;
//                        packed rows with groups of 4 query heads run their
//                        products on the matrix cores.
//   merge_kernel         log-sum-exp merge of the splits of one query head
//                        (partials arrive rotated back), current token,
//                        normalisation.
//   score / softmax / accumulate kernels   the three stages of the
//                        reference's split path, for profiling and the op API.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <string>
#include <type_traits>

#include "torque_hip.h"
#include "tq_device.hpp"

using namespace tq;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TQ_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  g_last_error.clear();
  return TQ_OK;
}

bool valid_bits(int b) { return b == 2 || b == 3 || b == 4; }
bool valid_head_dim(int d) { return d == 64 || d == 128 || d == 256; }

int check_geometry(int head_dim, int bits) {
  if (!valid_head_dim(head_dim))
    return fail(TQ_ERR_UNSUPPORTED, "Unsupported head dimension: " + std::to_string(head_dim));
  if (bits != 0 && !valid_bits(bits)) return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
  return TQ_OK;
}

int packed_words(int head_dim, int bits) { return (head_dim * bits + 31) / 32; }

float sqrt_f32(int head_dim) { return static_cast<float>(std::sqrt(static_cast<double>(head_dim))); }

constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale threshold for the online softmax, in log2 units: the running
// reference maximum is only raised when a score exceeds it by more than this,
// so partial weights stay below 2^8.
constexpr float kRescaleThreshold = 8.0f;
constexpr int kMaxSplits = 256;
constexpr int kTokensPerIter = 2;  // tokens per lane group per loop iteration
constexpr int kWideTokensPerIter = 3;  // the same, in the instances of wide_iter_shape
constexpr int kPrefetchIters = 1;  // loop iterations whose loads are in flight ahead
constexpr int kScoreChains = 2;    // independent score product chains per token (matrix-core mode)
constexpr bool kPhaseFences = true;  // matrix-core mode: no interleaving of products with VALU work

// ============================================================== rotation


template <int D, typename T>
__global__ __launch_bounds__(kBlock) void fwht_kernel(const T* __restrict__ x, float* __restrict__ y, int64_t rows,
                                                      const float* __restrict__ s_first,
                                                      const float* __restrict__ s_second, float sqrt_d) {
  constexpr int E = D / kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefront exits together
  const int lane = lane_id();
  float v[E];
  const T* src = x + row * D + lane * E;
#pragma unroll
  for (int i = 0; i < E; ++i) v[i] = to_f32(src[i]);
  wave_rotate<D>(v, s_first, s_second, sqrt_d);
  float* dst = y + row * D + lane * E;
#pragma unroll
  for (int i = 0; i < E; ++i) dst[i] = v[i];
}

// ============================================================== append


// One wavefront per (row, stream).  Items [0, rows) are keys, [rows, 2 rows)
// values (when `streams` == 2).  Rows are (l, h, t) in [L, Hkv, seq_new] order.
// SCALED (per-vector scales): the rotated row x is quantized as x / s with
// s = sqrt(mean(x^2)) (1 for a zero row); s is stored at the token's slot of
// the [L, Hkv, capacity] scale slab, or multiplied into the dequantized
// values.
template <int D, int BITS, typename T, bool DEQUANT, bool SCALED>
__global__ __launch_bounds__(kBlock) void append_kernel(
    const T* __restrict__ keys, const T* __restrict__ values, int64_t rows, int streams, int64_t seq_new,
    int rotate_keys, int rotate_values, const float* __restrict__ signs_left, const float* __restrict__ signs_right,
    float sqrt_d, const float* __restrict__ key_bnd, const float* __restrict__ value_bnd,
    const float* __restrict__ key_cent, const float* __restrict__ value_cent, uint32_t* __restrict__ key_codes,
    uint32_t* __restrict__ value_codes, int64_t capacity, int64_t offset, float* __restrict__ key_out,
    float* __restrict__ value_out, float* __restrict__ key_scales, float* __restrict__ value_scales) {
  constexpr int E = D / kWave;
  constexpr int W = D * BITS / 32;
  __shared__ uint8_t s_codes[kWavesPerBlock][D];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave;
  const bool active = item < rows * streams;
  const bool is_v = item >= rows;
  const int64_t r = is_v ? item - rows : item;
  float scale = 1.f;  // per-vector scale (SCALED)
  if (active) {
    const T* src = (is_v ? values : keys) + r * D + lane * E;
    float v[E];
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = to_f32(src[i]);
    if (is_v ? rotate_values : rotate_keys) wave_rotate<D>(v, signs_right, signs_left, sqrt_d);
    const float* bnd = is_v ? value_bnd : key_bnd;
    if constexpr (SCALED) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) ss = fmaf(v[i], v[i], ss);
      ss = group_sum<kWave>(ss);
      const float rms = sqrtf(ss / static_cast<float>(D));
      scale = rms > 0.f ? rms : 1.f;
#pragma unroll
      for (int i = 0; i < E; ++i) v[i] = v[i] / scale;
    }
    if constexpr (DEQUANT) {
      const float* cent = is_v ? value_cent : key_cent;
      float* dst = (is_v ? value_out : key_out) + r * D + lane * E;
#pragma unroll
      for (int i = 0; i < E; ++i) dst[i] = SCALED ? cent[quantize_count<BITS>(v[i], bnd)] * scale
                                                  : cent[quantize_count<BITS>(v[i], bnd)];
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) s_codes[wave][lane * E + i] = static_cast<uint8_t>(quantize_count<BITS>(v[i], bnd));
    }
  }
  if constexpr (!DEQUANT) {
    __syncthreads();
    if (active && lane < W) {
      const uint32_t word = pack_word<BITS, D>(s_codes[wave], lane);
      const int64_t lh = r / seq_new, t = r - lh * seq_new;
      uint32_t* dst = (is_v ? value_codes : key_codes) + (lh * capacity + offset + t) * W + lane;
      *dst = word;
      if (SCALED && lane == 0) (is_v ? value_scales : key_scales)[lh * capacity + offset + t] = scale;
    }
  }
}

// ============================================================== unpack


// scales (or null): per-token scale slab [groups, capacity] multiplied in.
template <int BITS>
__global__ __launch_bounds__(kBlock) void unpack_kernel(const uint32_t* __restrict__ codes, int64_t groups,
                                                        int64_t capacity, int64_t seq_len, int head_dim,
                                                        const float* __restrict__ cent,
                                                        const float* __restrict__ scales, float* __restrict__ out) {
  const int W = head_dim * BITS / 32;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t total = groups * seq_len * head_dim;
  if (idx >= total) return;
  const int d = static_cast<int>(idx % head_dim);
  const int64_t tok = idx / head_dim;
  const int64_t g = tok / seq_len, t = tok - g * seq_len;
  const uint32_t* row = codes + (g * capacity + t) * W;
  const float c = cent[unpack_code<BITS>(row, d)];
  out[idx] = scales != nullptr ? c * scales[g * capacity + t] : c;
}

// ============================================================== decode


struct DecodeArgs {
  const void* q;
  int q_f16;
  const uint8_t* k;  // slab [L, Hkv, cap, row_bytes]
  const uint8_t* v;
  int64_t cap;
  int64_t seq_len;
  int num_layers, query_heads, kv_heads, group, n_hgroups;
  const float* cent_k;
  const float* cent_v;
  const float* signs_left;
  const float* signs_right;
  float sqrt_d;
  float q_scale;  // log2(e) / sqrt(D): scores come out in log2 units
  int rotate_query, inverse_output;
  // Append mode (new_k != null): the token new_k/new_v [L, Hkv, D] (float16
  // when new_f16, else float32) is rotated, quantized and packed into the
  // slabs at row seq_len by the split-0 workgroups, and joins the softmax as
  // the current token.
  const void* new_k;
  const void* new_v;
  int new_f16;
  const float* bnd_k;
  const float* bnd_v;
  uint32_t* k_slab;
  uint32_t* v_slab;
  int rotate_new_k, rotate_new_v;
  const float* cur_k;  // [L, Hkv, D] or null
  const float* cur_v;
  int n_splits;
  // Splits that read rows: n_splits, or in append mode n_splits - 1 when
  // split 0 (which also packs the new token) takes no rows and the others
  // cover every block with no more blocks each than a deal over all splits.
  int row_splits;
  float* ws_ml;   // [L * Hq, n_splits, 2]  (max, sum) of each split, log2 units
  float* ws_acc;  // [L * Hq, n_splits, D]  value accumulator of each split
  float* ws_cur_s; // [L * Hq]              score of the current token (log2 units)
  float* ws_cur_v; // [L * Hkv, D]          current token's value, rotated back when requested
  float* out;     // [L, Hq, D]
  // Per-vector scales (SCALED kernels): [L, Hkv, cap] float32 per stream; a
  // token's score is multiplied by its key scale, its value by its value
  // scale.
  const float* k_scales;
  const float* v_scales;
  int wide_iter;  // host side only: launch the kWideTokensPerIter instance
};

// Finish one output row held by a wavefront: optional extra dense token
// (decode-with-current), normalisation, optional inverse rotation, store.
// A[D]: accumulator relative to max M (log2 units), L: softmax sum.
template <int D>
__device__ __forceinline__ void finish_row(const float* A, float M, float L, const float* qs, const float* ck,
                                           const float* cv, int inverse, const float (&sg_left)[D / kWave],
                                           const float (&sg_right)[D / kWave], float sqrt_d, float* dst) {
  constexpr int E = D / kWave;
  const int lane = lane_id();
  float e[E];
#pragma unroll
  for (int i = 0; i < E; ++i) e[i] = A[lane * E + i];
  if (ck != nullptr) {
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) dot = fmaf(qs[lane * E + i], ck[lane * E + i], dot);
    dot = group_sum<kWave>(dot);
    const float mn = fmaxf(M, dot);
    const float f_old = L > 0.f ? fast_exp2(M - mn) : 0.f;
    const float f_cur = fast_exp2(dot - mn);
#pragma unroll
    for (int i = 0; i < E; ++i) e[i] = e[i] * f_old + cv[lane * E + i] * f_cur;
    L = L * f_old + f_cur;
  }
#pragma unroll
  for (int i = 0; i < E; ++i) e[i] = L > 0.f ? e[i] / L : 0.f;
  if (inverse) wave_rotate_signs<D>(e, sg_left, sg_right, sqrt_d);
#pragma unroll
  for (int i = 0; i < E; ++i) dst[lane * E + i] = e[i];
}

// One reduce-scatter step over lane pairs (i, i xor LM): the lower lane of a
// pair gets x_i + x_partner, the upper lane y_i + y_partner.
template <int LM>
__device__ __forceinline__ float scatter_pair(float x, float y, int lane) {
  if constexpr (LM == 16 || LM == 32) {
    const LanePair r = permlane_swap<LM>(x, y);
    return r.first + r.second;
  } else if constexpr (LM == 8) {
    const float sx = x + dpp_move<kDppRor8>(x);
    const float sy = y + dpp_move<kDppRor8>(y);
    return (lane & 8) ? sy : sx;
  } else {
    const bool upper = (lane & LM) != 0;
    const float send = upper ? x : y;
    const float keep = upper ? y : x;
    return keep + xor_partner<LM>(send, lane);
  }
}

// Reduce-scatter of buf[0, 2*LEN) over the lanes that differ in lane bits
// LM, LM/2, ..., LO (one step per bit, highest first): each step halves the
// live length, the upper lane of a pair keeping the upper half.  Afterwards a
// lane holds, summed over its partners, the chunk of the original buffer that
// its lane bits LO..LM select (bit LM weighs half the buffer).
template <int LO, int LM, int LEN, int NV>
__device__ __forceinline__ void reduce_scatter(float (&buf)[NV], int lane) {
#pragma unroll
  for (int k = 0; k < LEN; ++k) buf[k] = scatter_pair<LM>(buf[k], buf[k + LEN], lane);
  if constexpr (LM > LO) reduce_scatter<LO, LM / 2, LEN / 2, NV>(buf, lane);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Matrix-core score products leave on lane l, register i, the partial score
// of token 4 * ((l / 4) / LPT) + i over slice (l / 4) % LPT.  Sum over the
// LPT slices (lane bits 2 .. 2 + log2(LPT) - 1) and keep on lane l the token
// of its value layout, l / LPT, i.e. register (l / LPT) % 4: a reduce-scatter
// over lane bits log2(LPT) + 1 and log2(LPT) (which select that register)
// and an all-reduce over the slice bits below them.
template <int LPT>
__device__ __forceinline__ float slice_sum_select(f32x4 c, int lane) {
  static_assert(LPT == 4 || LPT == 8 || LPT == 16, "4, 8 or 16 slices per token");
  float buf[4] = {c[0], c[1], c[2], c[3]};
  reduce_scatter<LPT, 2 * LPT, 2, 4>(buf, lane);
  float v = buf[0];
  if constexpr (LPT >= 8) v += xor_partner<4>(v, lane);
  if constexpr (LPT >= 16) v += xor_partner<8>(v, lane);
  return v;
}

// U: tokens per lane group per loop iteration -- kTokensPerIter, or
// kWideTokensPerIter in the instances wide_iter_instance() names.
template <class Fmt, int D, int HG, bool QF16, bool SCALED, int U = kTokensPerIter>
__global__ __launch_bounds__(kBlock, 2) void decode_kernel(const DecodeArgs a) {
  constexpr int SD = Fmt::kSliceDims;
  constexpr int LPT = D / SD;        // lanes per token
  constexpr int TPW = kWave / LPT;   // tokens (lane groups) per wavefront
  constexpr int TPB = kWavesPerBlock * TPW;
  constexpr int PF = kPrefetchIters;
  constexpr int NB = PF + 1;         // ring of iteration slots
  constexpr int STRIDE = U * TPB;    // tokens per workgroup iteration
  constexpr int E = D / kWave;
  constexpr int ROW = Fmt::template row_bytes<D>();
  constexpr int NV = HG * SD;        // accumulator values per lane
  using Raw = typename Fmt::Raw;

  __shared__ typename Fmt::LutT s_lut[2][Fmt::kLutEntries];
  __shared__ float s_q[HG][D];
  __shared__ float s_red[kWavesPerBlock][HG * D];
  __shared__ float s_mw[kWavesPerBlock][HG];
  __shared__ float s_lw[kWavesPerBlock][HG];
  // append mode: the new token's dequantized rotated key / value, and its codes
  __shared__ float s_cur[2][Fmt::kHasLut ? D : 1];
  __shared__ uint8_t s_codes[2][Fmt::kHasLut ? D : 1];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int gi = lane / LPT, slice = lane % LPT;

  // ---- work item.  Consecutive workgroup ids land on different XCDs
  // (round robin over 8); remap so the splits of one head group are
  // dispatched to the same XCD and share its L2.  XCD x receives the ids
  // x, x + 8, ...: nblk / 8 of them, one more for x < nblk % 8, and takes
  // that many consecutive work items starting at x (nblk / 8) + min(x,
  // nblk % 8), so every work item is taken exactly once for any nblk
  // (3 head groups x 170 splits: float32-kernel median 12.4-12.6 ->
  // 12.0-12.1 us against the remap only for multiples of 8).
  const int units = a.num_layers * a.kv_heads * a.n_hgroups;
  const int64_t nblk = static_cast<int64_t>(units) * a.n_splits;
  int64_t g = blockIdx.x;
  g = (g & 7) * (nblk >> 3) + min(g & 7, nblk & 7) + (g >> 3);
  const int unit = static_cast<int>(g / a.n_splits);
  const int split = static_cast<int>(g - static_cast<int64_t>(unit) * a.n_splits);
  const int lkv = unit / a.n_hgroups;
  const int hg = unit - lkv * a.n_hgroups;
  const int layer = lkv / a.kv_heads, kvh = lkv - layer * a.kv_heads;
  const int qh0 = kvh * a.group + hg * HG;

  // ---- tokens of this wavefront.  The sequence is cut into blocks of
  // STRIDE rows (one workgroup iteration) dealt out cyclically: split s takes
  // blocks s, s + n_splits, s + 2 n_splits, ..., so at any moment the splits
  // of a head group read neighbouring blocks (one contiguous window of
  // n_splits blocks per stream) rather than n_splits separate streams, which
  // keeps HBM rows open (measured: main loop 10.0 -> 9.0 us at M).  In
  // iteration i, lane group gi takes tokens first + gi + u * TPB + i * BSTRIDE
  // (u < U): one wavefront load covers TPW consecutive rows.  Token offsets
  // are 32-bit (the host keeps capacity * ROW below 2^31).  Every block but
  // the sequence's last is full.
  //
  // In append mode split 0 also quantizes the new token and finishes its
  // score and value, which sets the kernel's end when it reads rows too.  So
  // the rows go to splits 1.. only (deal index split - 1 over row_splits =
  // n_splits - 1) where that gives no split more blocks than a deal over
  // all of them, and split 0 deals past the last block; otherwise split 0
  // takes the lightest share (the one split n_splits - 1 would take) and
  // splits 1.. the shares of splits 0.. (24-layer 8K decode loop at 64
  // splits: 320 -> 289 us per step for the lightest share, 274 -> 249 for
  // none).
  const int t1 = static_cast<int>(a.seq_len);
  const int n_blocks = (t1 + STRIDE - 1) / STRIDE;
  const bool app_deal = Fmt::kHasLut && a.new_k != nullptr;
  const int row_splits = app_deal ? a.row_splits : a.n_splits;  // splits that read rows
  const int deal = !app_deal ? split : split > 0 ? split - 1 : row_splits < a.n_splits ? n_blocks : a.n_splits - 1;
  const int64_t t0 = static_cast<int64_t>(deal) * STRIDE;
  const int BSTRIDE = row_splits * STRIDE;
  const int first = static_cast<int>(t0) + wave * TPW;
  const int n_iter = deal < n_blocks ? (n_blocks - deal + row_splits - 1) / row_splits : 0;  // uniform per workgroup
  const uint8_t* kbase = a.k + static_cast<int64_t>(lkv) * a.cap * ROW;
  const uint8_t* vbase = a.v + static_cast<int64_t>(lkv) * a.cap * ROW;

  // Iteration i reads through buffer resources over rows
  // [t0 + i * STRIDE, t1): the workgroup-uniform part of a row's offset sits
  // in the resource base (scalar arithmetic), the lane's part in a fixed
  // per-token offset, and rows past the end of the split read as zeros and
  // are masked out when processed, so loads need no clamp and no branch.
  //
  // Matrix-core mode (packed rows, groups of 4 query heads): scores and value
  // updates run as 4x4x1 fp32 outer products (v_mfma_f32_4x4x1_16b_f32, 16
  // blocks of 4 lanes; block b = lanes 4b..4b+3, output element (i, j) of a
  // block in register i of lane 4b + j, A operand of row i from lane 4b + i,
  // B operand of column j from lane 4b + j).  Key rows are then read in a
  // second lane layout: a lane quad holds 4 consecutive tokens of one slice
  // (lane l: token 4 * ((l / 4) / LPT) + l % 4, slice (l / 4) % LPT), so one
  // product per slice dimension gives 4 tokens x 4 heads of partial scores.
  // Value rows keep the token-major layout (lane l: token l / LPT, slice
  // l % LPT), where a quad holds 4 slices of one token and one product per
  // slice dimension adds weight(head i) x value(dim of lane j).
  constexpr bool kMfma = Fmt::kHasLut && HG == 4;
  const int tk = kMfma ? 4 * ((lane >> 2) / LPT) + (lane & 3) : gi;
  const int sk = kMfma ? (lane >> 2) % LPT : slice;
  int lane_off_k[U], lane_off_v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    lane_off_k[u] = (wave * TPW + u * TPB + tk) * ROW + Fmt::slice_offset(sk);
    lane_off_v[u] = (wave * TPW + u * TPB + gi) * ROW + Fmt::slice_offset(slice);
  }
  // Every iteration's loads are issued unconditionally -- an iteration past
  // the end of the split gets an empty range and reads zeros without touching
  // memory -- so the compiler can count the loads in flight and wait only for
  // the iteration being processed, not for the prefetched ones.
  auto iter_rsrc = [&](const uint8_t* base, int i) {
    const int64_t row0 = min(t0 + static_cast<int64_t>(i) * BSTRIDE, static_cast<int64_t>(t1));
    return make_rsrc(base + row0 * ROW, static_cast<uint32_t>(t1 - row0) * ROW);
  };
  auto load_k = [&](int i, Raw (&kr)[U]) {
    const BufferRsrc rk = iter_rsrc(kbase, i);
#pragma unroll
    for (int u = 0; u < U; ++u) kr[u] = Fmt::load(rk, lane_off_k[u]);
  };
  auto load_v = [&](int i, Raw (&vr)[U]) {
    const BufferRsrc rv = iter_rsrc(vbase, i);
#pragma unroll
    for (int u = 0; u < U; ++u) vr[u] = Fmt::load(rv, lane_off_v[u]);
  };
  // Scaled mode: the key and value scales of the lane's value tokens
  // (lane group gi), loaded with the rows they belong to.
  const float* ksbase = SCALED ? a.k_scales + static_cast<int64_t>(lkv) * a.cap : nullptr;
  const float* vsbase = SCALED ? a.v_scales + static_cast<int64_t>(lkv) * a.cap : nullptr;
  auto load_scales = [&](int i, float (&ks)[U], float (&vs)[U]) {
    const int64_t row0 = min(t0 + static_cast<int64_t>(i) * BSTRIDE, static_cast<int64_t>(t1));
    const uint32_t bytes = static_cast<uint32_t>(t1 - row0) * 4u;
    const BufferRsrc rk = make_rsrc(ksbase + row0, bytes), rv = make_rsrc(vsbase + row0, bytes);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int off = (wave * TPW + u * TPB + gi) * 4;
      ks[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rk, off, 0, kRowLoadPolicy));
      vs[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, kRowLoadPolicy));
    }
  };
  auto load_iter = [&](int i, Raw (&kr)[U], Raw (&vr)[U], float (&ks)[U], float (&vs)[U]) {
    load_k(i, kr);
    load_v(i, vr);
    if constexpr (SCALED) load_scales(i, ks, vs);
  };

  // ---- set-up loads first: this thread's centroid-table entry, the query
  // row and its rotation signs.  Loads complete in order, so waiting for
  // these below does not wait for the K/V rows requested after them.
  typename Fmt::LutT lut_kv[2];
  if constexpr (Fmt::kHasLut) {
    static_assert(Fmt::kLutEntries <= kBlock, "one table entry per thread");
    if (tid < Fmt::kLutEntries) {
      lut_kv[0] = Fmt::lut_entry(tid, a.cent_k);
      lut_kv[1] = Fmt::lut_entry(tid, a.cent_v);
    }
  }
  // Append mode: the split-0 workgroups quantize the new token (wavefront 0
  // the key, 1 the value) while their first K/V rows are in flight.
  const bool appending = Fmt::kHasLut && a.new_k != nullptr;
  const bool appender = appending && split == 0 && wave < 2;
  constexpr int kLevels = Fmt::kHasLut ? (1 << Fmt::kBits) - 1 : 1;
  float tok[E], bnd[kLevels];
  if (appender) {
    const int64_t toff = static_cast<int64_t>(lkv) * D + lane * E;
    const void* src = wave == 0 ? a.new_k : a.new_v;
#pragma unroll
    for (int i = 0; i < E; ++i)
      tok[i] = a.new_f16 ? __half2float(static_cast<const __half*>(src)[toff + i]) : static_cast<const float*>(src)[toff + i];
    const float* b = wave == 0 ? a.bnd_k : a.bnd_v;
#pragma unroll
    for (int k = 0; k < kLevels; ++k) bnd[k] = b[k];
  }

  // Query bits are loaded raw and converted after the K/V requests below, so
  // the conversion does not hold those requests back.
  // A lane's query values as raw 32-bit words: E floats, or (E + 1) / 2 words
  // of fp16 pairs.
  float qe[E], sg_first[E], sg_second[E];
  uint32_t qw[E];
  if (wave < HG) {
    const int64_t qoff = (static_cast<int64_t>(layer) * a.query_heads + qh0 + wave) * D + lane * E;
    if constexpr (!QF16) {
      const uint32_t* q = static_cast<const uint32_t*>(a.q) + qoff;
#pragma unroll
      for (int i = 0; i < E; ++i) qw[i] = q[i];
    } else if constexpr (E == 1) {
      qw[0] = static_cast<const unsigned short*>(a.q)[qoff];
    } else {
      const uint32_t* q = reinterpret_cast<const uint32_t*>(static_cast<const unsigned short*>(a.q) + qoff);
#pragma unroll
      for (int i = 0; i < E / 2; ++i) qw[i] = q[i];
    }
  }
  // Signs are kept in registers: the query rotation uses (right, left), the
  // inverse rotation of the result (left, right).
  if ((wave < HG && (a.rotate_query || a.inverse_output)) || appender) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      sg_first[i] = a.signs_right[lane * E + i];
      sg_second[i] = a.signs_left[lane * E + i];
    }
  }

  // Software pipeline over a ring of NB = PF + 1 iteration slots: the loads of
  // iteration i + PF are in flight while iteration i is processed.  The first
  // PF iterations are requested here, so their latency overlaps the set-up.
  Raw kr[NB][U], vr[NB][U];
  float ksr[NB][U], vsr[NB][U];  // scaled mode only
#pragma unroll
  for (int j = 0; j < PF; ++j) load_iter(j, kr[j], vr[j], ksr[j], vsr[j]);

  // ---- centroid tables
  if constexpr (Fmt::kHasLut) {
    if (tid < Fmt::kLutEntries) {
      s_lut[0][tid] = lut_kv[0];
      s_lut[1][tid] = lut_kv[1];
    }
  }

  // ---- append mode: rotate (as on append) and quantize the new token.
  if constexpr (Fmt::kHasLut) {
    if (appender) {
      if (wave == 1 ? a.rotate_new_v : a.rotate_new_k) wave_rotate_signs<D>(tok, sg_first, sg_second, a.sqrt_d);
#pragma unroll
      for (int i = 0; i < E; ++i) s_codes[wave][lane * E + i] = static_cast<uint8_t>(quantize_count<Fmt::kBits>(tok[i], bnd));
    }
  }

  // ---- queries: optional rotation (bit-identical to the reference), then
  // the softmax scale and log2(e) folded in, so scores are in log2 units.
  if (wave < HG) {
#pragma unroll
    for (int i = 0; i < E; ++i)
      qe[i] = QF16 ? __half2float(__ushort_as_half(static_cast<unsigned short>(qw[i / 2] >> (16 * (i % 2)))))
                   : __builtin_bit_cast(float, qw[i]);
    if (a.rotate_query) wave_rotate_signs<D>(qe, sg_first, sg_second, a.sqrt_d);
#pragma unroll
    for (int i = 0; i < E; ++i) s_q[wave][lane * E + i] = qe[i] * a.q_scale;
  }
  lds_barrier();  // LDS-only exchange: the prefetched rows stay in flight
  if constexpr (Fmt::kHasLut) {
    if (appender) {
      // Dequantized values through the centroid table (entry c holds centroid
      // c first); one head group writes the packed words (all compute them).
#pragma unroll
      for (int i = 0; i < E; ++i) s_cur[wave][lane * E + i] = Fmt::first_centroid(s_lut[wave][s_codes[wave][lane * E + i]]);
      constexpr int W = D * Fmt::kBits / 32;
      if (hg == 0 && lane < W) {
        uint32_t* dst = (wave == 0 ? a.k_slab : a.v_slab) + (static_cast<int64_t>(lkv) * a.cap + a.seq_len) * W + lane;
        *dst = pack_word<Fmt::kBits, D>(s_codes[wave], lane);
      }
    }
  }

  // ---- head slots.  With HG == 4 the softmax runs in quad mode
  // (see process): the lane at quad position q4 owns head q4 ^ slot_x -- it
  // sums that head's score, exponentiates it and keeps its softmax sum -- and
  // its per-head registers (query slice, accumulators, running maxima) hold,
  // in slot r, head ((q4 + r) & 3) ^ slot_x.  With that rotation the lane
  // that owns a head is reached by one fixed quad_perm rotation per slot, so
  // the quad reduction and the weight broadcast need no selects; slot_x = 3
  // in the odd quads of a token's lanes makes the row_half_mirror / row_mirror
  // partners (quad position p <-> 3 - p) own the same head.  Other modes use
  // slot r = head r.
  constexpr bool kQuad = HG == 4 && !kMfma;
  const int q4 = lane & 3;
  const int slot_x = (kQuad && LPT >= 8 && ((lane >> 2) & 1)) ? 3 : 0;
  auto head_of = [&](int r) { return kQuad ? (((q4 + r) & 3) ^ slot_x) : r; };

  float qv[HG][SD];
  if constexpr (!kMfma) {
#pragma unroll
    for (int r = 0; r < HG; ++r)
#pragma unroll
      for (int i = 0; i < SD; ++i) qv[r][i] = s_q[head_of(r)][slice * SD + i];
  }

  float m[HG], lsum[HG], acc[HG][SD];
#pragma unroll
  for (int r = 0; r < HG; ++r) {
    m[r] = -INFINITY;
    lsum[r] = 0.f;  // quad and matrix-core modes use lsum[0] for the lane's own head
#pragma unroll
    for (int i = 0; i < SD; ++i) acc[r][i] = 0.f;
  }

  // Matrix-core mode: the lane's query slice of head lane % 4 (the B operand
  // of the score products), and the value accumulators cv[k] = (head 0..3) at
  // dimension slice * SD + k.  m[0] and lsum[0] belong to head lane % 4 and
  // the lane's value token; m[0] is wavefront-wide per head.
  float qk[SD];
  f32x4 cv[SD];
  if constexpr (kMfma) {
#pragma unroll
    for (int k = 0; k < SD; ++k) {
      qk[k] = s_q[lane & 3][sk * SD + k];
      cv[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  const typename Fmt::LutT* lut_k = s_lut[0];
  const typename Fmt::LutT* lut_v = s_lut[1];

  // Matrix-core mode, three parts of an iteration.  score_products: the
  // 4 x 4 x 1 products of one iteration's key rows, kScoreChains independent
  // chains per token (dimension k goes to chain k % kScoreChains).
  // score_reduce: the chains and then the slices are summed and each lane
  // keeps the score of its own (head, value token).  softmax_values: online
  // softmax update and value products of one iteration.
  constexpr int SC = kScoreChains;
  // Matrix ops and VALU ops issued interleaved in one wavefront cost more on
  // this part than the two issued in separate runs (measured: 634 against
  // 453 cycles for 16 products and 32 FMAs at two wavefronts per SIMD), so
  // each phase is fenced off from the compiler's scheduler: table decode,
  // then the products, then the reductions.
  auto score_products = [&](const Raw (&kr)[U], f32x4 (&c)[U][SC]) {
    float x[U][SD];
#pragma unroll
    for (int u = 0; u < U; ++u) Fmt::decode(kr[u], sk, lut_k, x[u]);
    if constexpr (kPhaseFences) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int k = 0; k < SD; ++k)
        c[u][k % SC] = __builtin_amdgcn_mfma_f32_4x4x1f32(x[u][k], qk[k],
                                                          k < SC ? f32x4{0.f, 0.f, 0.f, 0.f} : c[u][k % SC], 0, 0, 0);
    if constexpr (kPhaseFences) __builtin_amdgcn_sched_barrier(0);
  };
  auto score_reduce = [&](f32x4 (&c)[U][SC], float (&s_own)[U]) {
    if constexpr (kMfma) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int w = SC / 2; w >= 1; w /= 2)
#pragma unroll
          for (int j = 0; j < w; ++j) c[u][j] += c[u][j + w];
        s_own[u] = slice_sum_select<LPT>(c[u][0], lane);
      }
    }
  };
  auto softmax_values = [&](const Raw (&vr)[U], const float (&s_own)[U], const float (&vs)[U], int i, auto full) {
    constexpr bool FULL = decltype(full)::value;
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) valid[u] = FULL || first + i * BSTRIDE + u * TPB + gi < t1;
    float xv[U][SD];
#pragma unroll
    for (int u = 0; u < U; ++u) Fmt::decode(vr[u], slice, lut_v, xv[u]);
    bool need = false;
#pragma unroll
    for (int u = 0; u < U; ++u) need = need || (valid[u] && s_own[u] > m[0] + kRescaleThreshold);
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      // A running maximum moves: one maximum per head over the wavefront
      // (lanes sharing lane % 4), accumulators of head r rescaled by the
      // factor of the lanes that hold head r.
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) mx = valid[u] ? fmaxf(mx, s_own[u]) : mx;
      mx = strided_reduce<4, OpMax>(mx);
      float alpha = 1.f;
      if (mx > m[0] + kRescaleThreshold) {
        alpha = fast_exp2(m[0] - mx);  // 0 before the first maximum: nothing accumulated yet
        m[0] = mx;
      }
      lsum[0] *= alpha;
      const float a0 = quad_broadcast_t<0>(alpha), a1 = quad_broadcast_t<1>(alpha);
      const float a2 = quad_broadcast_t<2>(alpha), a3 = quad_broadcast_t<3>(alpha);
#pragma unroll
      for (int k = 0; k < SD; ++k) cv[k] *= f32x4{a0, a1, a2, a3};
    }
    float p[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      p[u] = valid[u] ? fast_exp2(s_own[u] - m[0]) : 0.f;
      lsum[0] += p[u];
      if constexpr (SCALED) p[u] *= vs[u];  // the value products take weight x value scale
    }
    if constexpr (kPhaseFences) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int k = 0; k < SD; ++k) cv[k] = __builtin_amdgcn_mfma_f32_4x4x1f32(p[u], xv[u][k], cv[k], 0, 0, 0);
    if constexpr (kPhaseFences) __builtin_amdgcn_sched_barrier(0);
  };

  // Partial dot products of this lane's slice: part[u][s] for token u, slot s.
  auto partial_scores = [&](const Raw (&kr)[U], float (&part)[U][HG]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float x[SD];
      Fmt::decode(kr[u], slice, lut_k, x);
#pragma unroll
      for (int s = 0; s < HG; ++s) {
        float d = 0.f;
#pragma unroll
        for (int k = 0; k < SD; ++k) d = fmaf(qv[s][k], x[k], d);
        part[u][s] = d;
      }
    }
  };

  // One iteration: U tokens per lane group -- U x HG partial scores, their
  // reduction over the group's lanes, one online-softmax update per head and
  // U value updates.  FULL iterations skip the validity masks.
  auto process = [&](const Raw (&kr)[U], const Raw (&vr)[U], const float (&ks)[U], const float (&vs)[U], int i,
                     auto full) {
    constexpr bool FULL = decltype(full)::value;
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) valid[u] = FULL || first + i * BSTRIDE + u * TPB + gi < t1;
    float part[U][HG];
    partial_scores(kr, part);
    // Value rows are decoded (LDS table reads issued) before the softmax so
    // the table latency overlaps it.
    float xv[U][SD];
#pragma unroll
    for (int u = 0; u < U; ++u) Fmt::decode(vr[u], slice, lut_v, xv[u]);
    if constexpr (kQuad) {
      // Quad reduction: slot r of the lane r positions back holds this
      // lane's own head, so three rotations add the quad's partials; the
      // other quads of the group are added after.  Each lane then
      // exponentiates its head for both tokens, and the value update takes
      // the weight of slot r from the lane r positions ahead.
      float own[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        own[u] = cross_quad_sum<LPT>(part[u][0] + quad_rotate_from<1>(part[u][1]) + quad_rotate_from<2>(part[u][2]) +
                                     quad_rotate_from<3>(part[u][3]));
      if constexpr (SCALED) {
#pragma unroll
        for (int u = 0; u < U; ++u) own[u] *= ks[u];
      }
      bool need = false;
#pragma unroll
      for (int u = 0; u < U; ++u) need = need || (valid[u] && own[u] > m[0] + kRescaleThreshold);
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        // Some running maximum moves (first iteration, rare afterwards).
        // The maxima are kept wavefront-wide: slot r holds the same head on
        // every lane group, and one maximum per head over all the groups'
        // tokens moves far less often than one per group would.
#pragma unroll
        for (int r = 0; r < HG; ++r) {
          float mx = -INFINITY;
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const float v = quad_rotate_to(own[u], r);
            mx = valid[u] ? fmaxf(mx, v) : mx;
          }
          mx = strided_reduce<LPT, OpMax>(mx);
          if (mx > m[r] + kRescaleThreshold) {
            if (m[r] != -INFINITY) {  // nothing accumulated before the first maximum
              const float alpha = fast_exp2(m[r] - mx);
#pragma unroll
              for (int k = 0; k < SD; ++k) acc[r][k] *= alpha;
              if (r == 0) lsum[0] *= alpha;
            }
            m[r] = mx;
          }
        }
      }
      float p_own[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p_own[u] = valid[u] ? fast_exp2(own[u] - m[0]) : 0.f;
        lsum[0] += p_own[u];
        if constexpr (SCALED) p_own[u] *= vs[u];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int r = 0; r < HG; ++r) {
          const float p = quad_rotate_to(p_own[u], r);
#pragma unroll
          for (int k = 0; k < SD; ++k) acc[r][k] = fmaf(p, xv[u][k], acc[r][k]);
        }
    } else {
      // Every lane of the group reduces and exponentiates every pair.
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int s = 0; s < HG; ++s) part[u][s] = SCALED ? group_sum<LPT>(part[u][s]) * ks[u] : group_sum<LPT>(part[u][s]);
      // Wavefront-wide running maxima, moved only when some score passes
      // one by more than the threshold (as in quad mode).
      bool need = false;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int s = 0; s < HG; ++s) need = need || (valid[u] && part[u][s] > m[s] + kRescaleThreshold);
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
        for (int s = 0; s < HG; ++s) {
          float mx = -INFINITY;
#pragma unroll
          for (int u = 0; u < U; ++u) mx = valid[u] ? fmaxf(mx, part[u][s]) : mx;
          mx = strided_reduce<LPT, OpMax>(mx);
          if (mx > m[s] + kRescaleThreshold) {
            if (m[s] != -INFINITY) {  // nothing accumulated before the first maximum
              const float alpha = fast_exp2(m[s] - mx);
              lsum[s] *= alpha;
#pragma unroll
              for (int k = 0; k < SD; ++k) acc[s][k] *= alpha;
            }
            m[s] = mx;
          }
        }
      }
      float p[U][HG];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int s = 0; s < HG; ++s) {
          p[u][s] = valid[u] ? fast_exp2(part[u][s] - m[s]) : 0.f;
          lsum[s] += p[u][s];
          if constexpr (SCALED) p[u][s] *= vs[u];
        }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int s = 0; s < HG; ++s)
#pragma unroll
          for (int k = 0; k < SD; ++k) acc[s][k] = fmaf(p[u][s], xv[u][k], acc[s][k]);
    }
  };

  // The ring is unrolled NB times with no exit inside it, so the waits for
  // each slot are the same on every trip and leave the PF prefetched slots in
  // flight; loads for iterations past n_iter get an empty range and read
  // nothing, and their compute is skipped (a wavefront-uniform branch: the
  // longest splits of the 24-layer 8K decode loop run 3 iterations, not 4).
  for (int it = 0; it < n_iter; it += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = it + j;
      load_iter(i + PF, kr[(j + PF) % NB], vr[(j + PF) % NB], ksr[(j + PF) % NB], vsr[(j + PF) % NB]);
      if (j > 0 && i >= n_iter) continue;
      const bool full = first + i * BSTRIDE + (U - 1) * TPB + TPW <= t1;
      if constexpr (kMfma) {
        f32x4 c[U][SC];
        float s_own[U];
        score_products(kr[j], c);
        score_reduce(c, s_own);
        if constexpr (SCALED) {
#pragma unroll
          for (int u = 0; u < U; ++u) s_own[u] *= ksr[j][u];
        }
        if (full)
          softmax_values(vr[j], s_own, vsr[j], i, std::true_type{});
        else
          softmax_values(vr[j], s_own, vsr[j], i, std::false_type{});
      } else {
        if (full)
          process(kr[j], vr[j], ksr[j], vsr[j], i, std::true_type{});
        else
          process(kr[j], vr[j], ksr[j], vsr[j], i, std::false_type{});
      }
    }
  }

  // ---- combine the lane groups of this workgroup (log-sum-exp).
  // The running maxima are wavefront-wide: m[r] is the same on every lane
  // that holds the same head in slot r, and lane 0 holds head r in slot r.
  // So the lane groups' sums share one reference per head and add without
  // rescaling: the softmax sums over the lanes of one slice (in quad mode a
  // lane holds only its own head's sum and takes slot r's from the lane r
  // positions ahead; the sums are equal on the lanes of a group that hold the
  // same head in the same slot), the accumulators by a reduce-scatter.  The
  // wavefronts' partials are weighted against the workgroup maximum when
  // they are added after the barrier.
  if constexpr (kMfma) {
    // Matrix-core mode: lane l holds head l % 4 and value token l / LPT; the
    // LPT / 4 lanes of a token that hold the same head add each weight once.
    const float ls = (lane % LPT) < 4 ? lsum[0] : 0.f;
    const float lw = strided_reduce<4, OpSum>(ls);
    if (lane < 4) {
      s_mw[wave][lane] = m[0];
      s_lw[wave][lane] = lw;
    }
  } else {
#pragma unroll
    for (int r = 0; r < HG; ++r) {
      const float ls = !kQuad || r == 0 ? lsum[kQuad ? 0 : r] : quad_rotate_to(lsum[0], r);
      const float lw = strided_reduce<LPT, OpSum>(ls);
      if (lane == 0) {
        s_mw[wave][r] = m[r];
        s_lw[wave][r] = lw;
      }
    }
  }
  // Reduce-scatter the accumulators over the TPW lane groups of the
  // wavefront: afterwards lane (gi, slice) holds values
  // [gi * NV / TPW, (gi + 1) * NV / TPW) of its slice, summed over groups.
  {
    float buf[NV];
#pragma unroll
    for (int r = 0; r < HG; ++r)
#pragma unroll
      for (int k = 0; k < SD; ++k) buf[r * SD + k] = kMfma ? cv[k][r] : acc[r][k];
    if constexpr (TPW > 1) reduce_scatter<LPT, kWave / 2, NV / 2, NV>(buf, lane);
    constexpr int W = NV / TPW;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const int v = gi * W + k;
      const int r = v / SD, d = v - r * SD;
      s_red[wave][head_of(r) * D + slice * SD + d] = buf[k];
    }
  }
  __syncthreads();
  // Weight of each wavefront's partial for head h against the workgroup
  // maximum (zero for a wavefront that saw no token); returns that maximum.
  auto wave_weights = [&](int h, float (&f)[kWavesPerBlock]) {
    float M = s_mw[0][h];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) M = fmaxf(M, s_mw[w][h]);
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) f[w] = s_mw[w][h] == -INFINITY ? 0.f : fast_exp2(s_mw[w][h] - M);
    return M;
  };
  // Sum of the wavefronts' accumulators into s_red[0], weighted.
  auto combine_waves = [&]() {
    for (int o = tid; o < HG * D; o += kBlock) {
      float f[kWavesPerBlock];
      wave_weights(o / D, f);
      float v = s_red[0][o] * f[0];
#pragma unroll
      for (int w = 1; w < kWavesPerBlock; ++w) v = fmaf(s_red[w][o], f[w], v);
      s_red[0][o] = v;
    }
    __syncthreads();
  };

  // ---- one split: this workgroup holds the whole result and finishes it.
  const int64_t qhg0 = static_cast<int64_t>(layer) * a.query_heads + qh0;
  if (a.n_splits == 1) {
    combine_waves();
    if (wave < HG) {
      float f[kWavesPerBlock];
      const float M = wave_weights(wave, f);
      float l = 0.f;
#pragma unroll
      for (int w = 0; w < kWavesPerBlock; ++w) l = fmaf(s_lw[w][wave], f[w], l);
      const float* ck = appending ? s_cur[0] : a.cur_k ? a.cur_k + static_cast<int64_t>(lkv) * D : nullptr;
      const float* cv = appending ? s_cur[1] : a.cur_v ? a.cur_v + static_cast<int64_t>(lkv) * D : nullptr;
      finish_row<D>(&s_red[0][wave * D], M, l, s_q[wave], ck, cv, a.inverse_output, sg_second, sg_first, a.sqrt_d,
                    a.out + (qhg0 + wave) * D);
    }
    return;
  }

  // ---- several splits: publish this split's partial for merge_kernel.  The
  // accumulator is stored inverse-rotated already: the rotation is linear, so
  // the merge is a plain weighted sum per dimension.  Split 0 also publishes
  // the current token's score per query head and its value per KV head.
  // Wavefront h < HG sums head h's row over the 4 wavefronts' partials
  // straight from LDS (no combining pass, no second barrier).
  if (wave < HG) {
    float f[kWavesPerBlock];
    const float M = wave_weights(wave, f);
    float e[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      float v = s_red[0][wave * D + lane * E + i] * f[0];
#pragma unroll
      for (int w = 1; w < kWavesPerBlock; ++w) v = fmaf(s_red[w][wave * D + lane * E + i], f[w], v);
      e[i] = v;
    }
    if (a.inverse_output) wave_rotate_signs<D>(e, sg_second, sg_first, a.sqrt_d);
    float* dst = a.ws_acc + ((qhg0 + wave) * a.n_splits + split) * D + lane * E;
#pragma unroll
    for (int i = 0; i < E; ++i) dst[i] = e[i];
    if (lane == 0) {
      float l = 0.f;
#pragma unroll
      for (int w = 0; w < kWavesPerBlock; ++w) l = fmaf(s_lw[w][wave], f[w], l);
      a.ws_ml[((qhg0 + wave) * a.n_splits + split) * 2] = M;
      a.ws_ml[((qhg0 + wave) * a.n_splits + split) * 2 + 1] = l;
    }
    if (split == 0 && (appending || a.cur_k != nullptr)) {
      const float* ck = (appending ? s_cur[0] : a.cur_k + static_cast<int64_t>(lkv) * D) + lane * E;
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) dot = fmaf(s_q[wave][lane * E + i], ck[i], dot);
      dot = group_sum<kWave>(dot);
      if (lane == 0) a.ws_cur_s[qhg0 + wave] = dot;
      if (wave == 0 && hg == 0) {
        float v[E];
        const float* cv = (appending ? s_cur[1] : a.cur_v + static_cast<int64_t>(lkv) * D) + lane * E;
#pragma unroll
        for (int i = 0; i < E; ++i) v[i] = cv[i];
        if (a.inverse_output) wave_rotate_signs<D>(v, sg_second, sg_first, a.sqrt_d);
#pragma unroll
        for (int i = 0; i < E; ++i) a.ws_cur_v[static_cast<int64_t>(lkv) * D + lane * E + i] = v[i];
      }
    }
  }
}

#include "decode_mx.hpp"

// Log-sum-exp merge of the splits: M = max(max_s M_s, current score),
// L = sum_s L_s 2^(M_s - M) (+ 2^(score - M)), out = (sum_s A_s 2^(M_s - M)
// (+ 2^(score - M) value)) / L.  The split accumulators A_s are already
// rotated back, so every dimension is independent: one workgroup per (query
// head, kMergeDims dimensions), its threads split the splits into kMergeGroups
// strided groups and issue all their loads before the (max, sum) reduction.
constexpr int kMergeDims = 16;  // 16: M -0.6 us per step against 32 (8 equal, 64 +2 us)
constexpr int kMergeGroups = kBlock / kMergeDims;
constexpr int kMergePerThread = kMaxSplits / kMergeGroups;

struct MergeArgs {
  int query_heads, kv_heads, group, n_splits;
  const float* ws_ml;   // [L * Hq, n_splits, 2]
  const float* ws_acc;  // [L * Hq, n_splits, D]
  const float* cur_s;   // [L * Hq] or null
  const float* cur_v;   // [L * Hkv, D]
  float* out;           // [L, Hq, D]
};

template <int D>
__global__ __launch_bounds__(kBlock) void merge_kernel(const MergeArgs a) {
  constexpr int CH = D / kMergeDims;
  __shared__ float s_f[kMaxSplits];
  __shared__ float s_red[kWavesPerBlock];
  __shared__ float s_part[kMergeGroups][kMergeDims];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  // Same XCD remap as the split kernel: XCD x takes the x-th eighth of the
  // query heads, whose partials that kernel wrote through the same XCD's L2
  // (measured: C5 loop 336 -> 332 us per step, M unchanged).
  int64_t mb = blockIdx.x;
  const int64_t nmb = gridDim.x;
  mb = (mb & 7) * (nmb >> 3) + min(mb & 7, nmb & 7) + (mb >> 3);
  const int64_t qhg = mb / CH;
  const int c = static_cast<int>(mb - qhg * CH);
  const int ns = a.n_splits;
  const int d = tid % kMergeDims, grp = tid / kMergeDims;
  const float* ml = a.ws_ml + qhg * ns * 2;
  const float* acc = a.ws_acc + qhg * ns * D + c * kMergeDims + d;

  float vals[kMergePerThread];
#pragma unroll
  for (int k = 0; k < kMergePerThread; ++k) {
    const int sp = grp + k * kMergeGroups;
    vals[k] = sp < ns ? acc[static_cast<int64_t>(sp) * D] : 0.f;
  }
  const float ms = tid < ns ? ml[tid * 2] : -INFINITY;
  const float ls = tid < ns ? ml[tid * 2 + 1] : 0.f;
  float cs = -INFINITY;
  if (a.cur_s != nullptr) cs = a.cur_s[qhg];

  const float mx = group_reduce<kWave, OpMax>(ms);
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3])), cs);
  const float f = ls > 0.f ? fast_exp2(ms - M) : 0.f;
  if (tid < ns) s_f[tid] = f;
  const float lw = group_sum<kWave>(ls * f);
  __syncthreads();
  if (lane == 0) s_red[wave] = lw;
  float part = 0.f;
#pragma unroll
  for (int k = 0; k < kMergePerThread; ++k) {
    const int sp = grp + k * kMergeGroups;
    if (sp < ns) part = fmaf(vals[k], s_f[sp], part);
  }
  s_part[grp][d] = part;
  __syncthreads();
  if (tid < kMergeDims) {
    float L = s_red[0] + s_red[1] + s_red[2] + s_red[3];
    float v = s_part[0][d];
#pragma unroll
    for (int g = 1; g < kMergeGroups; ++g) v += s_part[g][d];
    if (a.cur_s != nullptr) {
      const int layer = static_cast<int>(qhg / a.query_heads);
      const int qh = static_cast<int>(qhg - static_cast<int64_t>(layer) * a.query_heads);
      const int64_t lkv = static_cast<int64_t>(layer) * a.kv_heads + qh / a.group;
      const float fc = fast_exp2(cs - M);
      v = fmaf(fc, a.cur_v[lkv * D + c * kMergeDims + d], v);
      L += fc;
    }
    a.out[qhg * D + c * kMergeDims + d] = L > 0.f ? v / L : 0.f;
  }
}

// ============================================================== split path stages


template <class Fmt, int D>
__global__ __launch_bounds__(kBlock) void score_kernel(const float* __restrict__ q, const uint8_t* __restrict__ codes,
                                                       int64_t seq_len, const float* __restrict__ cent,
                                                       float* __restrict__ scores) {
  constexpr int SD = Fmt::kSliceDims;
  constexpr int LPT = D / SD;
  constexpr int TPW = kWave / LPT;
  constexpr int ROW = Fmt::template row_bytes<D>();
  __shared__ typename Fmt::LutT s_lut[Fmt::kLutEntries];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int gi = lane / LPT, slice = lane % LPT;
  const int b = blockIdx.y;
  for (int e = tid; e < Fmt::kLutEntries; e += kBlock) s_lut[e] = Fmt::lut_entry(e, cent);
  __syncthreads();
  float qv[SD];
#pragma unroll
  for (int i = 0; i < SD; ++i) qv[i] = q[static_cast<int64_t>(b) * D + slice * SD + i];
  const int64_t t = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave) * TPW + gi;
  float x[SD];
  float s = 0.f;
  if (t < seq_len) {
    const auto r = Fmt::load(codes + (static_cast<int64_t>(b) * seq_len + t) * ROW, slice);
    Fmt::decode(r, slice, s_lut, x);
#pragma unroll
    for (int i = 0; i < SD; ++i) s = fmaf(qv[i], x[i], s);
  }
  s = group_sum<LPT>(s);
  if (t < seq_len && slice == 0) scores[static_cast<int64_t>(b) * seq_len + t] = s;
}

__global__ __launch_bounds__(kBlock) void softmax_kernel(const float* __restrict__ scores, int64_t seq_len,
                                                         float scale, float* __restrict__ w) {
  __shared__ float s_red[kWavesPerBlock];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const float* row = scores + static_cast<int64_t>(blockIdx.x) * seq_len;
  float* orow = w + static_cast<int64_t>(blockIdx.x) * seq_len;
  float mx = -INFINITY;
  for (int64_t t = tid; t < seq_len; t += kBlock) mx = fmaxf(mx, row[t] * scale);
  mx = group_reduce<kWave, OpMax>(mx);
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int64_t t = tid; t < seq_len; t += kBlock) sum += expf(row[t] * scale - mx);
  sum = group_sum<kWave>(sum);
  if (lane == 0) s_red[wave] = sum;
  __syncthreads();
  sum = s_red[0] + s_red[1] + s_red[2] + s_red[3];
  for (int64_t t = tid; t < seq_len; t += kBlock) orow[t] = expf(row[t] * scale - mx) / sum;
}

template <class Fmt, int D>
__global__ __launch_bounds__(kBlock) void accumulate_kernel(const float* __restrict__ w,
                                                            const uint8_t* __restrict__ codes, int64_t seq_len,
                                                            const float* __restrict__ cent, float* __restrict__ out) {
  constexpr int SD = Fmt::kSliceDims;
  constexpr int LPT = D / SD;
  constexpr int TPW = kWave / LPT;
  constexpr int TPB = kWavesPerBlock * TPW;
  constexpr int ROW = Fmt::template row_bytes<D>();
  __shared__ typename Fmt::LutT s_lut[Fmt::kLutEntries];
  __shared__ float s_part[TPB][D];  // one row per lane group: summed in a fixed order
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int gi = lane / LPT, slice = lane % LPT;
  const int b = blockIdx.x;
  for (int e = tid; e < Fmt::kLutEntries; e += kBlock) s_lut[e] = Fmt::lut_entry(e, cent);
  __syncthreads();
  float acc[SD];
#pragma unroll
  for (int i = 0; i < SD; ++i) acc[i] = 0.f;
  float x[SD];
  for (int64_t t = wave * TPW + gi; t < seq_len; t += TPB) {
    const float wt = w[static_cast<int64_t>(b) * seq_len + t];
    const auto r = Fmt::load(codes + (static_cast<int64_t>(b) * seq_len + t) * ROW, slice);
    Fmt::decode(r, slice, s_lut, x);
#pragma unroll
    for (int i = 0; i < SD; ++i) acc[i] = fmaf(wt, x[i], acc[i]);
  }
#pragma unroll
  for (int i = 0; i < SD; ++i) s_part[wave * TPW + gi][slice * SD + i] = acc[i];
  __syncthreads();
  for (int d = tid; d < D; d += kBlock) {
    float v = 0.f;
    for (int r = 0; r < TPB; ++r) v += s_part[r][d];
    out[static_cast<int64_t>(b) * D + d] = v;
  }
}

// ============================================================== measurement


constexpr int kStreamThreads = 512;  // streaming-read probe: 512 threads, one workgroup per CU

// Streaming-read probe (the bench's HBM ceiling): every thread keeps four
// nontemporal 16-byte loads in flight over a grid-stride pass.  The shape is
// the best of a sweep on MI355X (grid-stride and per-workgroup chunks; 1, 2,
// 4, 8, 16 loads in flight; 256 / 512 / 1024 threads; 1-16 workgroups per
// CU; with and without the nontemporal bit): 6.9-7.0 TB/s over a 768 MiB
// pass, against 6.3-6.5 for the best cached-load shapes.  The store happens
// only if the xor of everything read equals a fixed pattern, which keeps the
// loads live without writing in practice.
__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(const uint4* __restrict__ p, int64_t n16,
                                                                     float* __restrict__ sink) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kStreamThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kStreamThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(q + i), b = __builtin_nontemporal_load(q + i + stride);
    const u32x4 c = __builtin_nontemporal_load(q + i + 2 * stride), d = __builtin_nontemporal_load(q + i + 3 * stride);
    const u32x4 x = a ^ b ^ c ^ d;
    acc ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  for (; i < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(q + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = 1.f;
}

// ============================================================== host helpers


int pick_hg(int group) {
  if (group % 4 == 0) return 4;
  if (group % 2 == 0) return 2;
  return 1;
}

// The split kernel a decode call runs: the float32 kernel (decode_kernel,
// 4x4x1 fp32 matrix products or VALU FMAs, 256 threads, two workgroups per
// CU) or, for 4-bit packed rows in groups of 4 query heads at head_dim 64 or
// 128, decode_mx_kernel (16x16x32 products of exact f16 splits, 768 threads,
// one workgroup per CU) unless TQ_F32_PRODUCTS asks for the former.
enum class SplitKernel { Fp32, Mx };

struct Plan {
  int hg, n_hgroups, units, n_splits;
  SplitKernel kernel;
  int block_rows;  // rows per workgroup iteration (the unit the sequence is dealt out in)
  int tokens_per_iter;  // decode_kernel: tokens per lane group per iteration
};

constexpr int kMinTokensPerSplit = 128;

int default_splits(int units, int64_t seq_len, int num_cus, int wgs_per_cu) {
  if (num_cus <= 0) num_cus = 256;
  const int64_t target = static_cast<int64_t>(wgs_per_cu) * num_cus;
  // Whole waves only: rounding target / units up would overshoot the target
  // when units does not divide it, and the few workgroups past it run as a
  // second wave.  Measured on MI355X, 3 head groups x 64K tokens: matrix
  // kernel 86 splits 16.6-17.1 us against 11.3-11.9 at 85, float32 kernel
  // 171 splits 15.3-16.0 us against 12.8-13.5 at 170.
  int64_t ns = std::max<int64_t>(1, target / units);
  const int64_t by_len = std::max<int64_t>(1, (seq_len + kMinTokensPerSplit - 1) / kMinTokensPerSplit);
  ns = std::min(ns, by_len);
  // A length cap just above one workgroup per CU (8192 + t tokens over 4 KV
  // heads: 65 splits, 260 workgroups) leaves a few CUs running two, and
  // those end the kernel late; one workgroup per CU with an extra block on
  // a few splits ends sooner.  Measured on MI355X, a 4 x 8192-token layer:
  // 10.0 us per decode at 64 splits, 11.2 at 63 (four splits with an extra
  // block), 12.6 at 65 (260 workgroups); a 24-layer 8K decode loop 375 ->
  // 340 us per step.
  if (units * ns > num_cus && units * ns <= num_cus + num_cus / 8)
    ns = std::max<int64_t>(1, num_cus / units);
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, kMaxSplits));
  return static_cast<int>(ns);
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

// Workspace layout: [ml: Lq * ns * 2][acc: Lq * ns * D][cur_s: Lq][cur_v: Lkv * D]
// floats, Lq = layers * query heads, Lkv = layers * KV heads, each section
// 256-byte aligned.
struct WsLayout {
  size_t ml, acc, cur_s, cur_v, total;
};

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

WsLayout workspace_layout(int64_t lq, int64_t lkv, int head_dim, int n_splits) {
  WsLayout w;
  w.ml = 0;
  w.acc = align256(static_cast<size_t>(lq) * n_splits * 2 * sizeof(float));
  w.cur_s = w.acc + align256(static_cast<size_t>(lq) * n_splits * head_dim * sizeof(float));
  w.cur_v = w.cur_s + align256(static_cast<size_t>(lq) * sizeof(float));
  w.total = w.cur_v + align256(static_cast<size_t>(lkv) * head_dim * sizeof(float));
  return w;
}

// ---- static scratch of the no-allocation decode entry point.
// One array per GPU in device memory, held until the process ends; every
// tq_decode_noalloc call on a GPU uses that GPU's copy as its split-K
// workspace (which needs no initialisation: each call writes every partial it
// later reads), so calls that overlap on one GPU race.  In host code
// `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
constexpr size_t kScratchBytes = size_t(8) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address in *out (looked up on the first call
// on that device), or an error code with the message set.  The lookup is not a stream
// operation, but it may load the code object, which a stream capture does not
// allow: a first call on a device made inside a capture is refused with a
// message, before anything is enqueued.
int device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    return fail(TQ_ERR_LAUNCH, std::string("tq_decode_noalloc: no current HIP device: ") + hipGetErrorString(e));
  }
  if (dev < 0 || dev >= kMaxDevices) {
    return fail(TQ_ERR_UNSUPPORTED, "tq_decode_noalloc: device index " + std::to_string(dev) + " out of range");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
      return fail(TQ_ERR_BAD_ARG, "tq_decode_noalloc: the first call on device " + std::to_string(dev) +
                                      " is inside a stream capture; make one call on that device outside capture first");
    }
    void* ptr = nullptr;
    const hipError_t r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (r != hipSuccess || ptr == nullptr) {
      return fail(TQ_ERR_LAUNCH, std::string("tq_decode_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                                     hipGetErrorString(r));
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TQ_OK;
}

// Rows per workgroup iteration of decode_kernel for `fmt` (2/3/4 packed
// bits, 16 dense fp16, 32 dense fp32): tokens per lane group x lane groups
// per wavefront (64 / (D / slice dims)) x wavefronts; packed slices hold 16
// dimensions, fp16 rows 8, fp32 rows 4.
int decode_block_rows(int fmt, int head_dim, int tokens_per_iter = kTokensPerIter) {
  const bool packed = fmt == 2 || fmt == 3 || fmt == 4;
  const int slice_dims = packed ? 16 : (fmt == 16 ? 8 : 4);
  return tokens_per_iter * kWavesPerBlock * kWave * slice_dims / head_dim;
}

// decode_kernel also has instances with kWideTokensPerIter tokens per lane
// group for 4-bit rows at head_dim 256 in groups of 4 query heads (48 rows
// per workgroup iteration against 32; 211 VGPRs, no spills).
template <class Fmt, int D, int HG>
constexpr bool wide_iter_instance() {
  return std::is_same_v<Fmt, PackedB4> && D == 256 && HG == 4;
}
bool wide_iter_shape(int fmt, int head_dim, int hg) { return fmt == 4 && head_dim == 256 && hg == 4; }

// Tokens per lane group per iteration of a decode_kernel call over seq_len
// rows and at most `ns_cap` splits.  Two measurements on MI355X (4 KV heads,
// 64 splits) put a wide iteration at about 1.6 narrow ones: at 8193-8320
// rows (5 iterations of 32 rows on the longest split against 3 of 48) a
// 24-layer decode loop takes 275 against 289 us per step, at 8192 rows (4
// against 3) one layer 11.2 against 10.0 us.  So the wide instance runs
// where 1.6 x its iterations stay below the narrow count: where the last
// narrow iteration is a nearly empty one, not on long sequences.
int fp32_tokens_per_iter(int fmt, int head_dim, int hg, int64_t seq_len, int64_t ns_cap) {
  if (!wide_iter_shape(fmt, head_dim, hg)) return kTokensPerIter;
  auto iters = [&](int u) {
    const int64_t rows = decode_block_rows(fmt, head_dim, u);
    const int64_t blocks = std::max<int64_t>(1, (seq_len + rows - 1) / rows);
    const int64_t ns = std::max<int64_t>(1, std::min(blocks, ns_cap));
    return (blocks + ns - 1) / ns;
  };
  return 8 * iters(kWideTokensPerIter) < 5 * iters(kTokensPerIter) ? kWideTokensPerIter : kTokensPerIter;
}

// Shapes the matrix-core split kernel takes: groups of 4 query heads with
// 4-bit rows at head_dim 64 / 128 / 256 or 2-bit rows at head_dim 128.
bool mx_shape(int fmt, int head_dim, int hg) {
  return hg == 4 && ((fmt == 4 && (head_dim == 64 || head_dim == 128 || head_dim == 256)) ||
                     (fmt == 2 && head_dim == 128));
}

// Fewest 128-row blocks per split at which the matrix-core kernel runs by
// default.  Measured on MI355X (wall time per decode, each kernel on its own
// default split plan): at head_dim 128 it is level with the float32 kernel at
// 2 blocks per split and ahead from 4 (0.6 us at 16K tokens x 8 KV heads,
// 1.6 us at 32K); at head_dim 256 it trails at 1-4 blocks (0.2-1.6 us) and
// leads at 8 (2.5 us at 64K x 4 and 128K x 2).  With less work per
// workgroup, writing its 128 KB of tables costs more than its loop saves.
int mx_min_blocks_per_split(int head_dim) { return head_dim == 256 ? 8 : 4; }

// Split kernel and split count of a decode over `units` work units with
// decode `flags` (n_splits <= 0: the default count for the chosen kernel).
struct KernelChoice {
  SplitKernel kernel;
  int n_splits;
};
KernelChoice choose_kernel(int units, int64_t seq_len, int n_splits, int fmt, int head_dim, int hg, int flags,
                           int num_cus) {
  if (mx_shape(fmt, head_dim, hg) && (flags & TQ_F32_PRODUCTS) == 0) {
    const int ns = n_splits > 0 ? n_splits : default_splits(units, seq_len, num_cus, 1);
    const int64_t blocks = std::max<int64_t>(1, (seq_len + mx::kStride - 1) / mx::kStride);
    if ((flags & TQ_MATRIX_PRODUCTS) != 0 || blocks / std::min<int64_t>(blocks, ns) >= mx_min_blocks_per_split(head_dim))
      return {SplitKernel::Mx, ns};
  }
  return {SplitKernel::Fp32, n_splits > 0 ? n_splits : default_splits(units, seq_len, num_cus, 2)};
}

// Fills the split plan of a decode call over `fmt` rows (see
// decode_block_rows) with decode `flags`; every split gets at least one block.
int make_plan(int num_layers, int kv_heads, int query_heads, int64_t seq_len, int n_splits, int fmt, int head_dim,
              int flags, Plan* p) {
  if (num_layers <= 0 || kv_heads <= 0 || query_heads <= 0)
    return fail(TQ_ERR_BAD_ARG, "num_layers, kv_heads and query_heads must be positive");
  if (query_heads % kv_heads != 0)
    return fail(TQ_ERR_BAD_ARG, "query head count " + std::to_string(query_heads) + " must be divisible by kv_heads " +
                                    std::to_string(kv_heads));
  if (seq_len < 0) return fail(TQ_ERR_BAD_ARG, "seq_len must be non-negative");
  const int group = query_heads / kv_heads;
  p->hg = pick_hg(group);
  p->n_hgroups = group / p->hg;
  // One launch holds at most 2^32 - 1 work-items: units x splits workgroups.
  const int64_t max_wg = ((int64_t(1) << 32) - 1) / kBlock;
  const int64_t units = static_cast<int64_t>(num_layers) * kv_heads * p->n_hgroups;
  if (units > max_wg)
    return fail(TQ_ERR_BAD_ARG, "num_layers x kv_heads x head groups exceeds one launch; decode fewer layers per call");
  p->units = static_cast<int>(units);
  if ((flags & TQ_F32_PRODUCTS) != 0 && (flags & TQ_MATRIX_PRODUCTS) != 0)
    return fail(TQ_ERR_BAD_ARG, "TQ_F32_PRODUCTS and TQ_MATRIX_PRODUCTS exclude each other");
  const KernelChoice kc = choose_kernel(p->units, seq_len, n_splits, fmt, head_dim, p->hg, flags, device_cu_count());
  p->kernel = kc.kernel;
  const int ns = kc.n_splits;
  if (ns > kMaxSplits) return fail(TQ_ERR_BAD_ARG, "n_splits must be at most " + std::to_string(kMaxSplits));
  p->tokens_per_iter = p->kernel == SplitKernel::Mx
                           ? 0
                           : fp32_tokens_per_iter(fmt, head_dim, p->hg, seq_len, std::min<int64_t>(ns, max_wg / units));
  p->block_rows = p->kernel == SplitKernel::Mx ? mx::kStride : decode_block_rows(fmt, head_dim, p->tokens_per_iter);
  const int64_t blocks = std::max<int64_t>(1, (seq_len + p->block_rows - 1) / p->block_rows);
  p->n_splits = static_cast<int>(std::min<int64_t>({blocks, static_cast<int64_t>(ns), max_wg / units}));
  return TQ_OK;
}

template <class Fmt, int D, int HG, bool QF16, bool SC, int U>
void launch_decode_u(const DecodeArgs& a, int nblk, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL((decode_kernel<Fmt, D, HG, QF16, SC, U>), dim3(nblk), dim3(kBlock), 0, stream, start, stop,
                          0, a);
  else
    hipLaunchKernelGGL((decode_kernel<Fmt, D, HG, QF16, SC, U>), dim3(nblk), dim3(kBlock), 0, stream, a);
}

template <class Fmt, int D, int HG, bool QF16, bool SC>
void launch_decode_q(const DecodeArgs& a, int nblk, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if constexpr (wide_iter_instance<Fmt, D, HG>()) {
    if (a.wide_iter) return launch_decode_u<Fmt, D, HG, QF16, SC, kWideTokensPerIter>(a, nblk, stream, start, stop);
  }
  launch_decode_u<Fmt, D, HG, QF16, SC, kTokensPerIter>(a, nblk, stream, start, stop);
}

// Scaled kernels exist for packed rows only (the host never passes scales
// with dense rows).
template <class Fmt, int D, int HG, bool QF16>
void launch_decode_s(const DecodeArgs& a, int nblk, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if constexpr (Fmt::kHasLut) {
    if (a.k_scales != nullptr) return launch_decode_q<Fmt, D, HG, QF16, true>(a, nblk, stream, start, stop);
  }
  launch_decode_q<Fmt, D, HG, QF16, false>(a, nblk, stream, start, stop);
}

template <class Fmt, int D, int HG>
void launch_decode(const DecodeArgs& a, int nblk, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (a.q_f16)
    launch_decode_s<Fmt, D, HG, true>(a, nblk, stream, start, stop);
  else
    launch_decode_s<Fmt, D, HG, false>(a, nblk, stream, start, stop);
}

template <class Fmt, int D>
int dispatch_hg(const DecodeArgs& a, int hg, int nblk, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
  switch (hg) {
    case 1:
      launch_decode<Fmt, D, 1>(a, nblk, s, e0, e1);
      break;
    case 2:
      launch_decode<Fmt, D, 2>(a, nblk, s, e0, e1);
      break;
    case 4:
      launch_decode<Fmt, D, 4>(a, nblk, s, e0, e1);
      break;
    default:
      return fail(TQ_ERR_UNSUPPORTED, "unsupported query-head group");
  }
  return TQ_OK;
}

template <class Fmt>
int dispatch_d(const DecodeArgs& a, int head_dim, int hg, int nblk, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
  switch (head_dim) {
    case 64:
      return dispatch_hg<Fmt, 64>(a, hg, nblk, s, e0, e1);
    case 128:
      return dispatch_hg<Fmt, 128>(a, hg, nblk, s, e0, e1);
    case 256:
      return dispatch_hg<Fmt, 256>(a, hg, nblk, s, e0, e1);
    default:
      return fail(TQ_ERR_UNSUPPORTED, "Unsupported head dimension: " + std::to_string(head_dim));
  }
}

// Common front end of tq_decode / tq_decode_dense.  fmt: 2/3/4 packed bits,
// 16 dense fp16, 32 dense fp32.
// The new token of tq_decode_append.
struct AppendSpec {
  const void* keys;
  const void* values;
  int dtype;  // TQ_F32 or TQ_F16
  const float* key_boundaries;
  const float* value_boundaries;
  int flags;  // TQ_ROTATE_KEYS | TQ_ROTATE_VALUES
};

int launch_fp32(const DecodeArgs& a, int fmt, int head_dim, int hg, int nblk, hipStream_t stream, hipEvent_t start,
                hipEvent_t stop);
struct ProfileEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
int launch_merge(const MergeArgs& m, int num_layers, int query_heads, int head_dim, hipStream_t stream,
                 bool profiled, const ProfileEvents* caller_events);

template <int D, bool QF16, int BITS>
void launch_mx_t(const DecodeArgs& a, dim3 grid, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL((decode_mx_kernel<D, QF16, BITS>), grid, dim3(mx::threads_of<D>()), 0, stream, start,
                          stop, 0, a);
  else
    hipLaunchKernelGGL((decode_mx_kernel<D, QF16, BITS>), grid, dim3(mx::threads_of<D>()), 0, stream, a);
}

template <int D, int BITS>
void launch_mx_d(const DecodeArgs& a, dim3 grid, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (a.q_f16)
    launch_mx_t<D, true, BITS>(a, grid, stream, start, stop);
  else
    launch_mx_t<D, false, BITS>(a, grid, stream, start, stop);
}

// Grid (split, head group, layer x KV head) of decode_mx_kernel.
int launch_mx(const DecodeArgs& a, int fmt, int head_dim, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  constexpr int kMaxGridYZ = 65535;
  const int lkv = a.num_layers * a.kv_heads;
  if (lkv > kMaxGridYZ || a.n_hgroups > kMaxGridYZ)
    return fail(TQ_ERR_BAD_ARG, "num_layers x kv_heads must be at most 65535 per call; decode fewer layers per call");
  const dim3 grid(a.n_splits, a.n_hgroups, lkv);
  if (fmt == 2 && head_dim == 128) {
    launch_mx_d<128, 2>(a, grid, stream, start, stop);
    return TQ_OK;
  }
  if (fmt != 4) return fail(TQ_ERR_UNSUPPORTED, "decode_mx_kernel: unsupported bit width " + std::to_string(fmt));
  switch (head_dim) {
    case 64:
      launch_mx_d<64, 4>(a, grid, stream, start, stop);
      return TQ_OK;
    case 128:
      launch_mx_d<128, 4>(a, grid, stream, start, stop);
      return TQ_OK;
    case 256:
      launch_mx_d<256, 4>(a, grid, stream, start, stop);
      return TQ_OK;
    default:
      return fail(TQ_ERR_UNSUPPORTED, "decode_mx_kernel: unsupported head dimension " + std::to_string(head_dim));
  }
}

int decode_common(int fmt, const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                  int head_dim, const void* keys, const void* values, int64_t capacity, int64_t seq_len,
                  const float* cent_k, const float* cent_v, const float* signs_left, const float* signs_right,
                  int flags, const float* cur_k, const float* cur_v, int n_splits, void* workspace,
                  size_t workspace_bytes, float* out, hipStream_t stream, hipEvent_t start, hipEvent_t stop,
                  const AppendSpec* app = nullptr,
                  const float* k_scales = nullptr, const float* v_scales = nullptr,
                  const ProfileEvents* merge_events = nullptr) {
  int rc = check_geometry(head_dim, 0);
  if (rc) return rc;
  if ((k_scales == nullptr) != (v_scales == nullptr))
    return fail(TQ_ERR_BAD_ARG, "key_scales and value_scales must both be given or both be null");
  if (k_scales != nullptr && app != nullptr)
    return fail(TQ_ERR_BAD_ARG, "per-vector scales are not supported by the fused append + decode");
  if (query == nullptr || out == nullptr || workspace == nullptr)
    return fail(TQ_ERR_BAD_ARG, "query, out and workspace must be non-null");
  if (query_dtype != TQ_F32 && query_dtype != TQ_F16) return fail(TQ_ERR_BAD_ARG, "query dtype must be F32 or F16");
  if (seq_len > 0 && (keys == nullptr || values == nullptr))
    return fail(TQ_ERR_BAD_ARG, "key and value slabs must be non-null");
  if (capacity < seq_len) return fail(TQ_ERR_BAD_ARG, "capacity must be >= seq_len");
  if ((cur_k == nullptr) != (cur_v == nullptr))
    return fail(TQ_ERR_BAD_ARG, "current_keys and current_values must both be given or both be null");
  if (app != nullptr) {
    if (app->keys == nullptr || app->values == nullptr || app->key_boundaries == nullptr ||
        app->value_boundaries == nullptr || keys == nullptr || values == nullptr)
      return fail(TQ_ERR_BAD_ARG, "new keys/values, boundaries and both slabs must be non-null");
    if (seq_len >= capacity) return fail(TQ_ERR_BAD_ARG, "slab is full: seq_len must be below capacity");
    if (app->dtype != TQ_F32 && app->dtype != TQ_F16) return fail(TQ_ERR_BAD_ARG, "new key/value dtype must be F32 or F16");
    if ((app->flags & (TQ_ROTATE_KEYS | TQ_ROTATE_VALUES)) && (signs_left == nullptr || signs_right == nullptr))
      return fail(TQ_ERR_BAD_ARG, "rotation flags need signs_left and signs_right");
  }
  if ((flags & (TQ_ROTATE_QUERY | TQ_INVERSE_OUTPUT)) && (signs_left == nullptr || signs_right == nullptr))
    return fail(TQ_ERR_BAD_ARG, "rotation flags need signs_left and signs_right");
  const bool packed = fmt == 2 || fmt == 3 || fmt == 4;
  if (packed && (cent_k == nullptr || cent_v == nullptr))
    return fail(TQ_ERR_BAD_ARG, "key and value centroids must be non-null");
  const int64_t row_bytes = packed ? static_cast<int64_t>(packed_words(head_dim, fmt)) * 4
                                   : static_cast<int64_t>(head_dim) * (fmt == 16 ? 2 : 4);
  if (capacity * row_bytes >= (1LL << 31))
    return fail(TQ_ERR_BAD_ARG, "capacity * row bytes must stay below 2 GiB per (layer, KV head)");
  Plan p;
  rc = make_plan(num_layers, kv_heads, query_heads, seq_len, n_splits, fmt, head_dim, flags, &p);
  if (rc) return rc;
  if (p.n_splits > 1 &&
      static_cast<int64_t>(num_layers) * query_heads * (head_dim / kMergeDims) > ((int64_t(1) << 32) - 1) / kBlock)
    return fail(TQ_ERR_BAD_ARG, "num_layers x query_heads exceeds one merge launch; decode fewer layers per call");

  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const WsLayout wl = workspace_layout(static_cast<int64_t>(num_layers) * query_heads,
                                      static_cast<int64_t>(num_layers) * kv_heads, head_dim, p.n_splits);
  if (workspace_bytes < wl.total)
    return fail(TQ_ERR_BAD_ARG, "workspace of " + std::to_string(workspace_bytes) + " bytes is smaller than the " +
                                    std::to_string(wl.total) + " bytes this call needs (" +
                                    std::to_string(p.n_splits) + " splits)");

  DecodeArgs a{};
  a.q = query;
  a.q_f16 = query_dtype == TQ_F16;
  a.k = static_cast<const uint8_t*>(keys);
  a.v = static_cast<const uint8_t*>(values);
  a.cap = capacity;
  a.seq_len = seq_len;
  a.num_layers = num_layers;
  a.query_heads = query_heads;
  a.kv_heads = kv_heads;
  a.group = query_heads / kv_heads;
  a.n_hgroups = p.n_hgroups;
  a.cent_k = cent_k;
  a.cent_v = cent_v;
  a.signs_left = signs_left;
  a.signs_right = signs_right;
  a.sqrt_d = sqrt_f32(head_dim);
  a.q_scale = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_dim)));
  a.rotate_query = (flags & TQ_ROTATE_QUERY) != 0;
  a.inverse_output = (flags & TQ_INVERSE_OUTPUT) != 0;
  a.cur_k = cur_k;
  a.cur_v = cur_v;
  a.k_scales = k_scales;
  a.v_scales = v_scales;
  if (app != nullptr) {
    a.new_k = app->keys;
    a.new_v = app->values;
    a.new_f16 = app->dtype == TQ_F16;
    a.bnd_k = app->key_boundaries;
    a.bnd_v = app->value_boundaries;
    a.k_slab = const_cast<uint32_t*>(static_cast<const uint32_t*>(keys));
    a.v_slab = const_cast<uint32_t*>(static_cast<const uint32_t*>(values));
    a.rotate_new_k = (app->flags & TQ_ROTATE_KEYS) != 0;
    a.rotate_new_v = (app->flags & TQ_ROTATE_VALUES) != 0;
  }
  a.n_splits = p.n_splits;
  a.row_splits = p.n_splits;
  if (app != nullptr && p.n_splits > 1) {
    // split 0 packs the new token; it reads no rows when the other splits
    // can take them all without a longer share
    const int64_t blocks = (seq_len + p.block_rows - 1) / p.block_rows;
    const int64_t n = p.n_splits;
    if ((blocks + n - 2) / (n - 1) <= (blocks + n - 1) / n) a.row_splits = p.n_splits - 1;
  }
  a.wide_iter = p.tokens_per_iter == kWideTokensPerIter;
  a.ws_ml = reinterpret_cast<float*>(ws + wl.ml);
  a.ws_acc = reinterpret_cast<float*>(ws + wl.acc);
  a.ws_cur_s = reinterpret_cast<float*>(ws + wl.cur_s);
  a.ws_cur_v = reinterpret_cast<float*>(ws + wl.cur_v);
  a.out = out;
  const int nblk = p.units * p.n_splits;
  MergeArgs m{};
  m.query_heads = query_heads;
  m.kv_heads = kv_heads;
  m.group = a.group;
  m.n_splits = p.n_splits;
  m.ws_ml = a.ws_ml;
  m.ws_acc = a.ws_acc;
  m.cur_s = (cur_k != nullptr || app != nullptr) ? a.ws_cur_s : nullptr;
  m.cur_v = a.ws_cur_v;
  m.out = out;

  if (p.kernel == SplitKernel::Mx) {
    rc = launch_mx(a, fmt, head_dim, stream, start, stop);
  } else {
    rc = launch_fp32(a, fmt, head_dim, p.hg, nblk, stream, start, stop);
  }
  if (rc) return rc;
  rc = launch_status("decode_kernel");
  if (rc || p.n_splits == 1) return rc;
  return launch_merge(m, num_layers, query_heads, head_dim, stream, start != nullptr || stop != nullptr, merge_events);
}

int launch_fp32(const DecodeArgs& a, int fmt, int head_dim, int hg, int nblk, hipStream_t stream, hipEvent_t start,
                hipEvent_t stop) {
  int rc;
  switch (fmt) {
    case 2:
      rc = dispatch_d<PackedB2>(a, head_dim, hg, nblk, stream, start, stop);
      break;
    case 3:
      rc = dispatch_d<PackedB3>(a, head_dim, hg, nblk, stream, start, stop);
      break;
    case 4:
      rc = dispatch_d<PackedB4>(a, head_dim, hg, nblk, stream, start, stop);
      break;
    case 16:
      rc = dispatch_d<DenseF16>(a, head_dim, hg, nblk, stream, start, stop);
      break;
    case 32:
      rc = dispatch_d<DenseF32>(a, head_dim, hg, nblk, stream, start, stop);
      break;
    default:
      return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(fmt));
  }
  return rc;
}

// Events of the merge launch of a timed call whose caller passes none, one
// pair per device (created on first use with that device current; never
// read, and shared by every stream of the device).  A timed call launches
// the merge kernel with profiling too: a dispatch launched with profiling
// events right after one launched without starts on six of the eight XCDs
// about 1.2 us after the other two (measured on MI355X for the split kernel
// after an unprofiled merge: median workgroup start skew 1.25 us, against
// 0.13 us with no events and 0.15 us with every dispatch profiled), and the
// split kernel's events would count that delay as its own time.
std::mutex g_profile_mutex;
ProfileEvents g_merge_events[kMaxDevices];

int merge_profile_events(ProfileEvents* ev) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TQ_ERR_LAUNCH, std::string("no current HIP device: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TQ_ERR_UNSUPPORTED, "device index " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(g_profile_mutex);
  ProfileEvents& p = g_merge_events[dev];
  if (p.start == nullptr) {
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t r = hipEventCreate(&a);
    if (r == hipSuccess) r = hipEventCreate(&b);
    if (r != hipSuccess) {
      if (a != nullptr) (void)hipEventDestroy(a);
      return fail(TQ_ERR_LAUNCH, std::string("hipEventCreate failed: ") + hipGetErrorString(r));
    }
    p.start = a;
    p.stop = b;
  }
  *ev = p;
  return TQ_OK;
}

template <int D>
void launch_merge_d(const MergeArgs& m, unsigned mblk, hipStream_t stream, const ProfileEvents* ev) {
  if (ev != nullptr)
    hipExtLaunchKernelGGL(merge_kernel<D>, dim3(mblk), dim3(kBlock), 0, stream, ev->start, ev->stop, 0, m);
  else
    hipLaunchKernelGGL(merge_kernel<D>, dim3(mblk), dim3(kBlock), 0, stream, m);
}

int launch_merge(const MergeArgs& m, int num_layers, int query_heads, int head_dim, hipStream_t stream,
                 bool profiled, const ProfileEvents* caller_events) {
  const unsigned mblk =
      static_cast<unsigned>(static_cast<int64_t>(num_layers) * query_heads * (head_dim / kMergeDims));
  ProfileEvents ev;
  if (caller_events != nullptr) {
    ev = *caller_events;
  } else if (profiled) {
    const int rc = merge_profile_events(&ev);
    if (rc) return rc;
  }
  const ProfileEvents* evp = (profiled || caller_events != nullptr) ? &ev : nullptr;
  switch (head_dim) {
    case 64:
      launch_merge_d<64>(m, mblk, stream, evp);
      break;
    case 128:
      launch_merge_d<128>(m, mblk, stream, evp);
      break;
    default:
      launch_merge_d<256>(m, mblk, stream, evp);
      break;
  }
  return launch_status("merge_kernel");
}

template <template <int> class Body, typename... Args>
int with_d(int head_dim, Args&&... args) {
  switch (head_dim) {
    case 64:
      return Body<64>::run(args...);
    case 128:
      return Body<128>::run(args...);
    case 256:
      return Body<256>::run(args...);
  }
  return fail(TQ_ERR_UNSUPPORTED, "Unsupported head dimension: " + std::to_string(head_dim));
}

// Workgroups per launch of the row kernels (fwht, append, unpack).  A HIP
// launch holds at most 2^32 - 1 work-items; larger calls are cut into
// launches of at most this many workgroups, in stream order.
constexpr int64_t kMaxLaunchBlocks = int64_t(1) << 20;

template <int D>
struct FwhtBody {
  static int run(const void* x, int x_dtype, float* y, int64_t rows, const float* s_first, const float* s_second,
                 hipStream_t stream) {
    const float sd = sqrt_f32(D);
    const int64_t chunk = kMaxLaunchBlocks * kWavesPerBlock;  // one wavefront per row
    for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
      const int64_t n = std::min(chunk, rows - r0);
      const unsigned nblk = static_cast<unsigned>((n + kWavesPerBlock - 1) / kWavesPerBlock);
      if (x_dtype == TQ_F16)
        hipLaunchKernelGGL((fwht_kernel<D, __half>), dim3(nblk), dim3(kBlock), 0, stream,
                           static_cast<const __half*>(x) + r0 * D, y + r0 * D, n, s_first, s_second, sd);
      else
        hipLaunchKernelGGL((fwht_kernel<D, float>), dim3(nblk), dim3(kBlock), 0, stream,
                           static_cast<const float*>(x) + r0 * D, y + r0 * D, n, s_first, s_second, sd);
      const int rc = launch_status("fwht_kernel");
      if (rc) return rc;
    }
    return TQ_OK;
  }
};

struct AppendParams {
  const void* keys;
  const void* values;
  int dtype;
  int64_t rows;
  int streams;
  int64_t seq_new;
  int rotate_keys, rotate_values;
  const float* signs_left;
  const float* signs_right;
  const float* key_bnd;
  const float* value_bnd;
  const float* key_cent;
  const float* value_cent;
  uint32_t* key_codes;
  uint32_t* value_codes;
  int64_t capacity, offset;
  float* key_out;
  float* value_out;
  bool dequant;
  // per-vector scales (scaled mode): scale slabs [L, Hkv, capacity] written
  // by the packing path; the dequantizing path multiplies them in.
  bool scaled;
  float* key_scales;
  float* value_scales;
};

// One launch over rows [g0 * seq_new + t0, + rows) of p: `groups` whole
// (layer, head) groups from group g0 (t0 = 0), or `rows` tokens of group g0
// from token t0.
template <int D, int BITS, typename T, bool DQ, bool SC>
int launch_append_part(const AppendParams& p, int64_t g0, int64_t t0, int64_t seq_part, int64_t rows,
                       hipStream_t stream) {
  constexpr int W = D * BITS / 32;
  const int64_t row0 = g0 * p.seq_new + t0;
  const int64_t nblk = (rows * p.streams + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL((append_kernel<D, BITS, T, DQ, SC>), dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0, stream,
                     static_cast<const T*>(p.keys) + row0 * D, static_cast<const T*>(p.values) + row0 * D, rows,
                     p.streams, seq_part, p.rotate_keys, p.rotate_values, p.signs_left, p.signs_right, sqrt_f32(D),
                     p.key_bnd, p.value_bnd, p.key_cent, p.value_cent,
                     p.key_codes ? p.key_codes + g0 * p.capacity * W : nullptr,
                     p.value_codes ? p.value_codes + g0 * p.capacity * W : nullptr, p.capacity, p.offset + t0,
                     p.key_out ? p.key_out + row0 * D : nullptr, p.value_out ? p.value_out + row0 * D : nullptr,
                     p.key_scales ? p.key_scales + g0 * p.capacity : nullptr,
                     p.value_scales ? p.value_scales + g0 * p.capacity : nullptr);
  return launch_status("append_kernel");
}

// rows = groups * seq_new items per stream; at most kMaxLaunchBlocks
// workgroups per launch, cut at whole groups, or at tokens when one group
// alone is larger.
template <int D, int BITS, typename T, bool DQ, bool SC>
int launch_append(const AppendParams& p, hipStream_t stream) {
  const int64_t max_rows = kMaxLaunchBlocks * kWavesPerBlock / p.streams;
  const int64_t groups = p.rows / p.seq_new;
  if (p.seq_new <= max_rows) {
    const int64_t per = max_rows / p.seq_new;
    for (int64_t g0 = 0; g0 < groups; g0 += per) {
      const int64_t ng = std::min(per, groups - g0);
      const int rc = launch_append_part<D, BITS, T, DQ, SC>(p, g0, 0, p.seq_new, ng * p.seq_new, stream);
      if (rc) return rc;
    }
    return TQ_OK;
  }
  for (int64_t g = 0; g < groups; ++g)
    for (int64_t t0 = 0; t0 < p.seq_new; t0 += max_rows) {
      const int64_t nt = std::min(max_rows, p.seq_new - t0);
      const int rc = launch_append_part<D, BITS, T, DQ, SC>(p, g, t0, nt, nt, stream);
      if (rc) return rc;
    }
  return TQ_OK;
}

template <int D, int BITS, typename T>
int append_mode(const AppendParams& p, hipStream_t stream) {
  if (p.scaled)
    return p.dequant ? launch_append<D, BITS, T, true, true>(p, stream) : launch_append<D, BITS, T, false, true>(p, stream);
  return p.dequant ? launch_append<D, BITS, T, true, false>(p, stream) : launch_append<D, BITS, T, false, false>(p, stream);
}

template <int D, int BITS>
int append_dtype(const AppendParams& p, hipStream_t stream) {
  return p.dtype == TQ_F16 ? append_mode<D, BITS, __half>(p, stream) : append_mode<D, BITS, float>(p, stream);
}

template <int D>
struct AppendBody {
  static int run(const AppendParams& p, int bits, hipStream_t stream) {
    switch (bits) {
      case 2:
        return append_dtype<D, 2>(p, stream);
      case 3:
        return append_dtype<D, 3>(p, stream);
      case 4:
        return append_dtype<D, 4>(p, stream);
      default:
        return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
    }
  }
};

template <int D>
struct StageBody {
  // op 0: score, op 2: accumulate
  template <class Fmt>
  static void go(int op, const float* a, const uint8_t* codes, int batch, int64_t seq_len, const float* cent,
                 float* out, hipStream_t stream) {
    constexpr int LPT = D / Fmt::kSliceDims;
    constexpr int TPB = kWavesPerBlock * (kWave / LPT);
    if (op == 0) {
      const int64_t nx = (seq_len + TPB - 1) / TPB;
      hipLaunchKernelGGL((score_kernel<Fmt, D>), dim3(static_cast<unsigned>(nx), batch), dim3(kBlock), 0, stream, a,
                         codes, seq_len, cent, out);
    } else {
      hipLaunchKernelGGL((accumulate_kernel<Fmt, D>), dim3(batch), dim3(kBlock), 0, stream, a, codes, seq_len, cent,
                         out);
    }
  }
  static int run(int op, int bits, const float* a, const uint8_t* codes, int batch, int64_t seq_len,
                 const float* cent, float* out, hipStream_t stream) {
    switch (bits) {
      case 2:
        go<PackedB2>(op, a, codes, batch, seq_len, cent, out, stream);
        break;
      case 3:
        go<PackedB3>(op, a, codes, batch, seq_len, cent, out, stream);
        break;
      case 4:
        go<PackedB4>(op, a, codes, batch, seq_len, cent, out, stream);
        break;
      default:
        return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
    }
    return launch_status(op == 0 ? "score_kernel" : "accumulate_kernel");
  }
};

template <int D>
struct UnpackBody {
  // One launch: `groups` groups of seq_len tokens (group stride `capacity`
  // rows) into out [groups, seq_len, D].
  template <int BITS>
  static int part(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, const float* cent,
                  const float* scales, float* out, hipStream_t stream) {
    const unsigned nblk = static_cast<unsigned>((groups * seq_len * D + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(unpack_kernel<BITS>, dim3(nblk), dim3(kBlock), 0, stream, codes, groups, capacity, seq_len, D,
                       cent, scales, out);
    return launch_status("unpack_kernel");
  }
  // At most kMaxLaunchBlocks workgroups (one thread per output value) per
  // launch: cut at whole groups, or at tokens when one group alone is larger.
  template <int BITS>
  static int chunks(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, const float* cent,
                    const float* scales, float* out, hipStream_t stream) {
    constexpr int W = D * BITS / 32;
    const int64_t max_tokens = kMaxLaunchBlocks * kBlock / D;
    if (seq_len <= max_tokens) {
      const int64_t per = max_tokens / seq_len;
      for (int64_t g0 = 0; g0 < groups; g0 += per) {
        const int64_t ng = std::min(per, groups - g0);
        const int rc = part<BITS>(codes + g0 * capacity * W, ng, capacity, seq_len, cent,
                                  scales ? scales + g0 * capacity : nullptr, out + g0 * seq_len * D, stream);
        if (rc) return rc;
      }
      return TQ_OK;
    }
    for (int64_t g = 0; g < groups; ++g)
      for (int64_t t0 = 0; t0 < seq_len; t0 += max_tokens) {
        const int64_t nt = std::min(max_tokens, seq_len - t0);
        const int rc = part<BITS>(codes + (g * capacity + t0) * W, 1, capacity, nt, cent,
                                  scales ? scales + g * capacity + t0 : nullptr, out + (g * seq_len + t0) * D, stream);
        if (rc) return rc;
      }
    return TQ_OK;
  }
  static int run(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, int bits,
                 const float* cent, const float* scales, float* out, hipStream_t stream) {
    switch (bits) {
      case 2:
        return chunks<2>(codes, groups, capacity, seq_len, cent, scales, out, stream);
      case 3:
        return chunks<3>(codes, groups, capacity, seq_len, cent, scales, out, stream);
      case 4:
        return chunks<4>(codes, groups, capacity, seq_len, cent, scales, out, stream);
      default:
        return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
    }
  }
};

int append_impl(const void* keys, const void* values, int dtype, int num_layers, int kv_heads, int64_t seq_new,
                int head_dim, int bits, const float* signs_left, const float* signs_right, int flags,
                const float* key_boundaries, const float* value_boundaries, uint32_t* key_codes,
                uint32_t* value_codes, int64_t capacity, int64_t offset, float* key_scales, float* value_scales,
                hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  if (num_layers <= 0 || kv_heads <= 0) return fail(TQ_ERR_BAD_ARG, "num_layers and kv_heads must be positive");
  if (seq_new < 0 || offset < 0) return fail(TQ_ERR_BAD_ARG, "seq_new and offset must be non-negative");
  if (offset + seq_new > capacity) return fail(TQ_ERR_BAD_ARG, "append past slab capacity");
  if (seq_new == 0) return TQ_OK;
  if (!keys || !values || !key_boundaries || !value_boundaries || !key_codes || !value_codes)
    return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  if ((flags & (TQ_ROTATE_KEYS | TQ_ROTATE_VALUES)) && (!signs_left || !signs_right))
    return fail(TQ_ERR_BAD_ARG, "rotation flags need signs_left and signs_right");
  if (dtype != TQ_F32 && dtype != TQ_F16) return fail(TQ_ERR_BAD_ARG, "dtype must be F32 or F16");
  AppendParams p{};
  p.keys = keys;
  p.values = values;
  p.dtype = dtype;
  p.rows = static_cast<int64_t>(num_layers) * kv_heads * seq_new;
  p.streams = 2;
  p.seq_new = seq_new;
  p.rotate_keys = (flags & TQ_ROTATE_KEYS) != 0;
  p.rotate_values = (flags & TQ_ROTATE_VALUES) != 0;
  p.signs_left = signs_left;
  p.signs_right = signs_right;
  p.key_bnd = key_boundaries;
  p.value_bnd = value_boundaries;
  p.key_codes = key_codes;
  p.value_codes = value_codes;
  p.capacity = capacity;
  p.offset = offset;
  p.scaled = key_scales != nullptr;
  p.key_scales = key_scales;
  p.value_scales = value_scales;
  return with_d<AppendBody>(head_dim, p, bits, stream);
}

int qdq_impl(const void* keys, const void* values, int dtype, int64_t rows, int head_dim, int bits,
             const float* signs_left, const float* signs_right, int flags, const float* key_boundaries,
             const float* value_boundaries, const float* key_centroids, const float* value_centroids,
             float* key_out, float* value_out, bool scaled, hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  if (rows < 0) return fail(TQ_ERR_BAD_ARG, "rows must be non-negative");
  if (rows == 0) return TQ_OK;
  if (!keys || !key_boundaries || !key_centroids || !key_out) return fail(TQ_ERR_BAD_ARG, "null key argument");
  const bool two = values != nullptr;
  if (two && (!value_boundaries || !value_centroids || !value_out))
    return fail(TQ_ERR_BAD_ARG, "null value argument");
  if ((flags & (TQ_ROTATE_KEYS | TQ_ROTATE_VALUES)) && (!signs_left || !signs_right))
    return fail(TQ_ERR_BAD_ARG, "rotation flags need signs_left and signs_right");
  if (dtype != TQ_F32 && dtype != TQ_F16) return fail(TQ_ERR_BAD_ARG, "dtype must be F32 or F16");
  AppendParams p{};
  p.keys = keys;
  p.values = two ? values : keys;
  p.dtype = dtype;
  p.rows = rows;
  p.streams = two ? 2 : 1;
  p.seq_new = rows;
  p.rotate_keys = (flags & TQ_ROTATE_KEYS) != 0;
  p.rotate_values = (flags & TQ_ROTATE_VALUES) != 0;
  p.signs_left = signs_left;
  p.signs_right = signs_right;
  p.key_bnd = key_boundaries;
  p.value_bnd = two ? value_boundaries : key_boundaries;
  p.key_cent = key_centroids;
  p.value_cent = two ? value_centroids : key_centroids;
  p.key_out = key_out;
  p.value_out = two ? value_out : key_out;
  p.dequant = true;
  p.scaled = scaled;
  return with_d<AppendBody>(head_dim, p, bits, stream);
}

int unpack_impl(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, int head_dim, int bits,
                const float* centroids, const float* scales, float* out, hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  if (groups < 0 || seq_len < 0 || capacity < seq_len) return fail(TQ_ERR_BAD_ARG, "bad unpack extents");
  if (groups == 0 || seq_len == 0) return TQ_OK;
  if (!codes || !centroids || !out) return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  return with_d<UnpackBody>(head_dim, codes, groups, capacity, seq_len, bits, centroids, scales, out, stream);
}

}  // namespace

// ============================================================== C ABI

extern "C" {

int tq_abi_version(void) { return TQ_ABI_VERSION; }

const char* tq_last_error(void) { return g_last_error.c_str(); }

int tq_fwht(const void* x, int x_dtype, float* y, int64_t rows, int head_dim, const float* signs_left,
            const float* signs_right, int inverse, hipStream_t stream) {
  int rc = check_geometry(head_dim, 0);
  if (rc) return rc;
  if (rows < 0) return fail(TQ_ERR_BAD_ARG, "rows must be non-negative");
  if (rows == 0) return TQ_OK;
  if (!x || !y || !signs_left || !signs_right) return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  if (x_dtype != TQ_F32 && x_dtype != TQ_F16) return fail(TQ_ERR_BAD_ARG, "x dtype must be F32 or F16");
  const float* first = inverse ? signs_left : signs_right;
  const float* second = inverse ? signs_right : signs_left;
  return with_d<FwhtBody>(head_dim, x, x_dtype, y, rows, first, second, stream);
}

int tq_quantize_pack(const float* values, int64_t rows, int head_dim, int bits, const float* boundaries,
                     uint32_t* packed, hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  if (rows < 0) return fail(TQ_ERR_BAD_ARG, "rows must be non-negative");
  if (rows == 0) return TQ_OK;
  if (!values || !boundaries || !packed) return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  AppendParams p{};
  p.keys = values;
  p.values = values;
  p.dtype = TQ_F32;
  p.rows = rows;
  p.streams = 1;
  p.seq_new = rows;
  p.key_bnd = boundaries;
  p.value_bnd = boundaries;
  p.key_codes = packed;
  p.value_codes = packed;
  p.capacity = rows;
  p.offset = 0;
  return with_d<AppendBody>(head_dim, p, bits, stream);
}

int tq_append(const void* keys, const void* values, int dtype, int num_layers, int kv_heads, int64_t seq_new,
              int head_dim, int bits, const float* signs_left, const float* signs_right, int flags,
              const float* key_boundaries, const float* value_boundaries, uint32_t* key_codes,
              uint32_t* value_codes, int64_t capacity, int64_t offset, hipStream_t stream) {
  return append_impl(keys, values, dtype, num_layers, kv_heads, seq_new, head_dim, bits, signs_left, signs_right, flags,
                     key_boundaries, value_boundaries, key_codes, value_codes, capacity, offset, nullptr, nullptr,
                     stream);
}

int tq_append_scaled(const void* keys, const void* values, int dtype, int num_layers, int kv_heads, int64_t seq_new,
                     int head_dim, int bits, const float* signs_left, const float* signs_right, int flags,
                     const float* key_boundaries, const float* value_boundaries, uint32_t* key_codes,
                     uint32_t* value_codes, float* key_scales, float* value_scales, int64_t capacity,
                     int64_t offset, hipStream_t stream) {
  if (key_scales == nullptr || value_scales == nullptr)
    return fail(TQ_ERR_BAD_ARG, "key_scales and value_scales must be non-null");
  return append_impl(keys, values, dtype, num_layers, kv_heads, seq_new, head_dim, bits, signs_left, signs_right, flags,
                     key_boundaries, value_boundaries, key_codes, value_codes, capacity, offset, key_scales,
                     value_scales, stream);
}

int tq_quantize_dequantize(const void* keys, const void* values, int dtype, int64_t rows, int head_dim, int bits,
                           const float* signs_left, const float* signs_right, int flags,
                           const float* key_boundaries, const float* value_boundaries,
                           const float* key_centroids, const float* value_centroids, float* key_out,
                           float* value_out, hipStream_t stream) {
  return qdq_impl(keys, values, dtype, rows, head_dim, bits, signs_left, signs_right, flags, key_boundaries,
                  value_boundaries, key_centroids, value_centroids, key_out, value_out, false, stream);
}

int tq_quantize_dequantize_scaled(const void* keys, const void* values, int dtype, int64_t rows, int head_dim,
                                  int bits, const float* signs_left, const float* signs_right, int flags,
                                  const float* key_boundaries, const float* value_boundaries,
                                  const float* key_centroids, const float* value_centroids, float* key_out,
                                  float* value_out, hipStream_t stream) {
  return qdq_impl(keys, values, dtype, rows, head_dim, bits, signs_left, signs_right, flags, key_boundaries,
                  value_boundaries, key_centroids, value_centroids, key_out, value_out, true, stream);
}

int tq_unpack_dequantize(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, int head_dim,
                         int bits, const float* centroids, float* out, hipStream_t stream) {
  return unpack_impl(codes, groups, capacity, seq_len, head_dim, bits, centroids, nullptr, out, stream);
}

int tq_unpack_dequantize_scaled(const uint32_t* codes, const float* scales, int64_t groups, int64_t capacity,
                                int64_t seq_len, int head_dim, int bits, const float* centroids, float* out,
                                hipStream_t stream) {
  if (scales == nullptr) return fail(TQ_ERR_BAD_ARG, "scales must be non-null");
  return unpack_impl(codes, groups, capacity, seq_len, head_dim, bits, centroids, scales, out, stream);
}

int tq_decode_default_splits(int num_layers, int kv_heads, int query_heads, int head_dim, int bits, int flags,
                             int64_t seq_len, int num_cus) {
  if (num_layers <= 0 || kv_heads <= 0 || query_heads <= 0 || query_heads % kv_heads != 0)
    return fail(TQ_ERR_BAD_ARG, "bad head configuration");
  if ((flags & TQ_F32_PRODUCTS) != 0 && (flags & TQ_MATRIX_PRODUCTS) != 0)
    return fail(TQ_ERR_BAD_ARG, "TQ_F32_PRODUCTS and TQ_MATRIX_PRODUCTS exclude each other");
  const int group = query_heads / kv_heads;
  const int hg = pick_hg(group);
  const int units = num_layers * kv_heads * (group / hg);
  if (num_cus <= 0) num_cus = device_cu_count();
  return choose_kernel(units, seq_len, 0, bits, head_dim, hg, flags, num_cus).n_splits;
}

const char* tq_decode_split_kernel(int num_layers, int kv_heads, int query_heads, int head_dim, int bits, int flags,
                                   int query_dtype, int64_t seq_len, int n_splits, int num_cus) {
  if (num_layers <= 0 || kv_heads <= 0 || query_heads <= 0 || query_heads % kv_heads != 0 ||
      !valid_head_dim(head_dim) || seq_len < 0) {
    fail(TQ_ERR_BAD_ARG, "bad head configuration");
    return nullptr;
  }
  const bool packed = bits == 2 || bits == 3 || bits == 4;
  if (!packed) {
    fail(TQ_ERR_UNSUPPORTED, "split kernel names cover packed rows (bits 2, 3, 4)");
    return nullptr;
  }
  if ((flags & TQ_F32_PRODUCTS) != 0 && (flags & TQ_MATRIX_PRODUCTS) != 0) {
    fail(TQ_ERR_BAD_ARG, "TQ_F32_PRODUCTS and TQ_MATRIX_PRODUCTS exclude each other");
    return nullptr;
  }
  const int group = query_heads / kv_heads;
  const int hg = pick_hg(group);
  const int units = num_layers * kv_heads * (group / hg);
  if (num_cus <= 0) num_cus = device_cu_count();
  static thread_local std::string name;
  const KernelChoice kc = choose_kernel(units, seq_len, n_splits, bits, head_dim, hg, flags, num_cus);
  if (kc.kernel == SplitKernel::Mx)
    name = "decode_mx_kernel<" + std::to_string(head_dim) + "," + (query_dtype == TQ_F16 ? "true" : "false") +
           (bits == 4 ? ">" : "," + std::to_string(bits) + ">");
  else if (fp32_tokens_per_iter(bits, head_dim, hg, seq_len, kc.n_splits) == kWideTokensPerIter)
    name = "decode_kernel<PackedB4,256,4," + std::to_string(kWideTokensPerIter) + ">";
  else
    name = "decode_kernel<PackedB" + std::to_string(bits) + "," + std::to_string(head_dim) + "," +
           std::to_string(hg) + ">";
  return name.c_str();
}

size_t tq_decode_workspace_bytes(int num_layers, int kv_heads, int query_heads, int head_dim, int n_splits,
                                 int num_cus) {
  if (num_layers <= 0 || kv_heads <= 0 || query_heads <= 0 || query_heads % kv_heads != 0) return 0;
  if (!valid_head_dim(head_dim)) return 0;
  const int group = query_heads / kv_heads;
  const int hg = pick_hg(group);
  const int units = num_layers * kv_heads * (group / hg);
  int ns = n_splits;
  // the larger of the two split kernels' defaults (two workgroups per CU)
  if (ns <= 0) ns = default_splits(units, static_cast<int64_t>(kMaxSplits) * kMinTokensPerSplit, num_cus, 2);
  ns = std::min(ns, kMaxSplits);
  return workspace_layout(static_cast<int64_t>(num_layers) * query_heads, static_cast<int64_t>(num_layers) * kv_heads,
                          head_dim, ns)
      .total;
}

int tq_decode(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads, int head_dim,
              int bits, const uint32_t* key_codes, const uint32_t* value_codes, int64_t capacity, int64_t seq_len,
              const float* key_centroids, const float* value_centroids, const float* signs_left,
              const float* signs_right, int flags, const float* current_keys, const float* current_values,
              int n_splits, void* workspace, size_t workspace_bytes, float* out, hipStream_t stream) {
  return tq_decode_timed(query, query_dtype, num_layers, query_heads, kv_heads, head_dim, bits, key_codes,
                         value_codes, capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right,
                         flags, current_keys, current_values, n_splits, workspace, workspace_bytes, out, stream,
                         nullptr, nullptr);
}

int tq_decode_noalloc(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                      int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                      int64_t capacity, int64_t seq_len, const float* key_centroids, const float* value_centroids,
                      const float* signs_left, const float* signs_right, int flags, const float* current_keys,
                      const float* current_values, int n_splits, float* out, hipStream_t stream) {
  if (!valid_bits(bits)) return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  // The split plan this call resolves to, and the scratch it needs, before
  // anything touches the device.
  Plan p;
  rc = make_plan(num_layers, kv_heads, query_heads, seq_len, n_splits, bits, head_dim, flags, &p);
  if (rc) return rc;
  const size_t need = workspace_layout(static_cast<int64_t>(num_layers) * query_heads,
                                       static_cast<int64_t>(num_layers) * kv_heads, head_dim, p.n_splits)
                          .total;
  if (need > kScratchBytes)
    return fail(TQ_ERR_BAD_ARG, "tq_decode_noalloc: this call needs " + std::to_string(need) +
                                    " bytes of scratch (" + std::to_string(p.n_splits) +
                                    " splits) but the static scratch holds " + std::to_string(kScratchBytes) +
                                    "; pass fewer splits or decode fewer layers per call");
  void* ws = nullptr;
  rc = device_scratch(stream, &ws);
  if (rc) return rc;
  return decode_common(bits, query, query_dtype, num_layers, query_heads, kv_heads, head_dim, key_codes,
                       value_codes, capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right, flags,
                       current_keys, current_values, p.n_splits, ws, kScratchBytes, out, stream, nullptr, nullptr);
}

int tq_decode_scaled(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads, int head_dim,
                     int bits, const uint32_t* key_codes, const uint32_t* value_codes, const float* key_scales,
                     const float* value_scales, int64_t capacity, int64_t seq_len, const float* key_centroids,
                     const float* value_centroids, const float* signs_left, const float* signs_right, int flags,
                     const float* current_keys, const float* current_values, int n_splits, void* workspace,
                     size_t workspace_bytes, float* out, hipStream_t stream) {
  return tq_decode_scaled_timed(query, query_dtype, num_layers, query_heads, kv_heads, head_dim, bits, key_codes,
                                value_codes, key_scales, value_scales, capacity, seq_len, key_centroids,
                                value_centroids, signs_left, signs_right, flags, current_keys, current_values,
                                n_splits, workspace, workspace_bytes, out, stream, nullptr, nullptr);
}

int tq_decode_scaled_timed(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                           int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                           const float* key_scales, const float* value_scales, int64_t capacity, int64_t seq_len,
                           const float* key_centroids, const float* value_centroids, const float* signs_left,
                           const float* signs_right, int flags, const float* current_keys,
                           const float* current_values, int n_splits, void* workspace, size_t workspace_bytes,
                           float* out, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (!valid_bits(bits)) return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
  if (seq_len > 0 && (key_scales == nullptr || value_scales == nullptr))
    return fail(TQ_ERR_BAD_ARG, "key_scales and value_scales must be non-null");
  // Per-vector scales multiply the softmax weights, which the f16-split
  // kernel cannot hold for a factor of unknown size: always float32 products.
  return decode_common(bits, query, query_dtype, num_layers, query_heads, kv_heads, head_dim, key_codes, value_codes,
                       capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right,
                       flags | TQ_F32_PRODUCTS, current_keys, current_values, n_splits, workspace, workspace_bytes,
                       out, stream, start, stop, nullptr,
                       seq_len > 0 ? key_scales : nullptr, seq_len > 0 ? value_scales : nullptr);
}

int tq_decode_append(const void* query, int query_dtype, const void* new_keys, const void* new_values, int kv_dtype,
                     int num_layers, int query_heads, int kv_heads, int head_dim, int bits, uint32_t* key_codes,
                     uint32_t* value_codes, int64_t capacity, int64_t seq_len, const float* key_centroids,
                     const float* value_centroids, const float* key_boundaries, const float* value_boundaries,
                     const float* signs_left, const float* signs_right, int append_flags, int decode_flags,
                     int n_splits, void* workspace, size_t workspace_bytes, float* out, hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  const AppendSpec app{new_keys, new_values, kv_dtype, key_boundaries, value_boundaries, append_flags};
  return decode_common(bits, query, query_dtype, num_layers, query_heads, kv_heads, head_dim, key_codes, value_codes,
                       capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right, decode_flags,
                       nullptr, nullptr, n_splits, workspace, workspace_bytes, out, stream, nullptr, nullptr, &app);
}

int tq_decode_timed(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                    int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                    int64_t capacity, int64_t seq_len, const float* key_centroids, const float* value_centroids,
                    const float* signs_left, const float* signs_right, int flags, const float* current_keys,
                    const float* current_values, int n_splits, void* workspace, size_t workspace_bytes, float* out,
                    hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (!valid_bits(bits)) return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
  return decode_common(bits, query, query_dtype, num_layers, query_heads, kv_heads, head_dim, key_codes,
                       value_codes, capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right, flags,
                       current_keys, current_values, n_splits, workspace, workspace_bytes, out, stream, start, stop);
}

int tq_decode_step_timed(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                         int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                         int64_t capacity, int64_t seq_len, const float* key_centroids, const float* value_centroids,
                         const float* signs_left, const float* signs_right, int flags, const float* current_keys,
                         const float* current_values, int n_splits, void* workspace, size_t workspace_bytes,
                         float* out, hipStream_t stream, hipEvent_t split_start, hipEvent_t split_stop,
                         hipEvent_t merge_start, hipEvent_t merge_stop) {
  if (!valid_bits(bits)) return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
  if ((merge_start == nullptr) != (merge_stop == nullptr))
    return fail(TQ_ERR_BAD_ARG, "merge_start and merge_stop must both be given or both be null");
  ProfileEvents mev;
  mev.start = merge_start;
  mev.stop = merge_stop;
  return decode_common(bits, query, query_dtype, num_layers, query_heads, kv_heads, head_dim, key_codes,
                       value_codes, capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right, flags,
                       current_keys, current_values, n_splits, workspace, workspace_bytes, out, stream, split_start,
                       split_stop, nullptr, nullptr, nullptr, merge_start != nullptr ? &mev : nullptr);
}

int tq_decode_dense(const void* query, int query_dtype, const void* keys, const void* values, int kv_dtype,
                    int num_layers, int query_heads, int kv_heads, int head_dim, int64_t capacity, int64_t seq_len,
                    const float* signs_left, const float* signs_right, int flags, int n_splits, void* workspace,
                    size_t workspace_bytes, float* out, hipStream_t stream) {
  return tq_decode_dense_timed(query, query_dtype, keys, values, kv_dtype, num_layers, query_heads, kv_heads,
                               head_dim, capacity, seq_len, signs_left, signs_right, flags, n_splits, workspace,
                               workspace_bytes, out, stream, nullptr, nullptr);
}

int tq_decode_dense_timed(const void* query, int query_dtype, const void* keys, const void* values, int kv_dtype,
                          int num_layers, int query_heads, int kv_heads, int head_dim, int64_t capacity,
                          int64_t seq_len, const float* signs_left, const float* signs_right, int flags,
                          int n_splits, void* workspace, size_t workspace_bytes, float* out, hipStream_t stream,
                          hipEvent_t start, hipEvent_t stop) {
  if (kv_dtype != TQ_F16 && kv_dtype != TQ_F32) return fail(TQ_ERR_BAD_ARG, "kv dtype must be F32 or F16");
  return decode_common(kv_dtype == TQ_F16 ? 16 : 32, query, query_dtype, num_layers, query_heads, kv_heads, head_dim,
                       keys, values, capacity, seq_len, nullptr, nullptr, signs_left, signs_right, flags, nullptr,
                       nullptr, n_splits, workspace, workspace_bytes, out, stream, start, stop);
}

int tq_score_packed(const float* query, const uint32_t* codes, int batch, int64_t seq_len, int head_dim, int bits,
                    const float* centroids, float* scores, hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  if (batch < 0 || seq_len < 0) return fail(TQ_ERR_BAD_ARG, "batch and seq_len must be non-negative");
  if (batch == 0 || seq_len == 0) return TQ_OK;
  if (!query || !codes || !centroids || !scores) return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  return with_d<StageBody>(head_dim, 0, bits, query, reinterpret_cast<const uint8_t*>(codes), batch, seq_len,
                           centroids, scores, stream);
}

int tq_softmax_rows(const float* scores, int batch, int64_t seq_len, float scale, float* weights,
                    hipStream_t stream) {
  if (batch < 0 || seq_len < 0) return fail(TQ_ERR_BAD_ARG, "batch and seq_len must be non-negative");
  if (batch == 0 || seq_len == 0) return TQ_OK;
  if (!scores || !weights) return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  hipLaunchKernelGGL(softmax_kernel, dim3(batch), dim3(kBlock), 0, stream, scores, seq_len, scale, weights);
  return launch_status("softmax_kernel");
}

int tq_accumulate_packed(const float* weights, const uint32_t* codes, int batch, int64_t seq_len, int head_dim,
                         int bits, const float* centroids, float* out, hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  if (batch < 0 || seq_len < 0) return fail(TQ_ERR_BAD_ARG, "batch and seq_len must be non-negative");
  if (batch == 0) return TQ_OK;
  if (!weights || !codes || !centroids || !out) return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  return with_d<StageBody>(head_dim, 2, bits, weights, reinterpret_cast<const uint8_t*>(codes), batch, seq_len,
                           centroids, out, stream);
}

int tq_stream_read(const void* data, size_t bytes, float* sink, int n_blocks, hipStream_t stream, hipEvent_t start,
                   hipEvent_t stop) {
  if (data == nullptr || sink == nullptr) return fail(TQ_ERR_BAD_ARG, "data and sink must be non-null");
  if (bytes % 16 != 0 || reinterpret_cast<uintptr_t>(data) % 16 != 0)
    return fail(TQ_ERR_BAD_ARG, "bytes and the data address must be multiples of 16");
  if (n_blocks <= 0) n_blocks = device_cu_count();
  const int64_t n16 = static_cast<int64_t>(bytes / 16);
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL(stream_read_kernel, dim3(n_blocks), dim3(kStreamThreads), 0, stream, start, stop, 0,
                          static_cast<const uint4*>(data), n16, sink);
  else
    hipLaunchKernelGGL(stream_read_kernel, dim3(n_blocks), dim3(kStreamThreads), 0, stream,
                       static_cast<const uint4*>(data), n16, sink);
  return launch_status("stream_read_kernel");
}

}  // extern "C"
