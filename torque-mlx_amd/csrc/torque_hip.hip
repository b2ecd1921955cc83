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
//                        (layer, KV head, query-head group) and one contiguous
//                        sequence split; the last workgroup of a group merges
//                        all splits (log-sum-exp) and applies the inverse
//                        rotation.  Fmt selects packed 2/3/4-bit or dense
//                        fp16/fp32 rows.
//   score / softmax / accumulate kernels   the three stages of the
//                        reference's split path, for profiling and the op API.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <string>

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
template <int D, int BITS, typename T, bool DEQUANT>
__global__ __launch_bounds__(kBlock) void append_kernel(
    const T* __restrict__ keys, const T* __restrict__ values, int64_t rows, int streams, int64_t seq_new,
    int rotate_keys, int rotate_values, const float* __restrict__ signs_left, const float* __restrict__ signs_right,
    float sqrt_d, const float* __restrict__ key_bnd, const float* __restrict__ value_bnd,
    const float* __restrict__ key_cent, const float* __restrict__ value_cent, uint32_t* __restrict__ key_codes,
    uint32_t* __restrict__ value_codes, int64_t capacity, int64_t offset, float* __restrict__ key_out,
    float* __restrict__ value_out) {
  constexpr int E = D / kWave;
  constexpr int W = D * BITS / 32;
  __shared__ uint8_t s_codes[kWavesPerBlock][D];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave;
  const bool active = item < rows * streams;
  const bool is_v = item >= rows;
  const int64_t r = is_v ? item - rows : item;
  if (active) {
    const T* src = (is_v ? values : keys) + r * D + lane * E;
    float v[E];
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = to_f32(src[i]);
    if (is_v ? rotate_values : rotate_keys) wave_rotate<D>(v, signs_right, signs_left, sqrt_d);
    const float* bnd = is_v ? value_bnd : key_bnd;
    if constexpr (DEQUANT) {
      const float* cent = is_v ? value_cent : key_cent;
      float* dst = (is_v ? value_out : key_out) + r * D + lane * E;
#pragma unroll
      for (int i = 0; i < E; ++i) dst[i] = cent[quantize_count<BITS>(v[i], bnd)];
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
    }
  }
}

// ============================================================== unpack


template <int BITS>
__global__ __launch_bounds__(kBlock) void unpack_kernel(const uint32_t* __restrict__ codes, int64_t groups,
                                                        int64_t capacity, int64_t seq_len, int head_dim,
                                                        const float* __restrict__ cent, float* __restrict__ out) {
  const int W = head_dim * BITS / 32;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t total = groups * seq_len * head_dim;
  if (idx >= total) return;
  const int d = static_cast<int>(idx % head_dim);
  const int64_t tok = idx / head_dim;
  const int64_t g = tok / seq_len, t = tok - g * seq_len;
  const uint32_t* row = codes + (g * capacity + t) * W;
  out[idx] = cent[unpack_code<BITS>(row, d)];
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
  const float* cur_k;  // [L, Hkv, D] or null
  const float* cur_v;
  int n_splits;
  int64_t split_len;
  unsigned* counters;  // [units]
  float2* ws_ml;       // [units, n_splits, HG]  (max, sum) per split
  float* ws_acc;       // [units, n_splits, HG, D]
  float* out;          // [L, Hq, D]
};

template <class Fmt, int D, int HG>
__global__ __launch_bounds__(kBlock, 2) void decode_kernel(const DecodeArgs a) {
  constexpr int SD = Fmt::kSliceDims;
  constexpr int LPT = D / SD;        // lanes per token
  constexpr int TPW = kWave / LPT;   // tokens per wavefront step
  constexpr int TPB = kWavesPerBlock * TPW;
  constexpr int U = kTokensPerIter;
  constexpr int E = D / kWave;
  constexpr int ROW = Fmt::template row_bytes<D>();
  using Raw = typename Fmt::Raw;

  __shared__ typename Fmt::LutT s_lut[2][Fmt::kLutEntries];
  __shared__ float s_q[HG][D];
  __shared__ float s_acc[HG][D];
  __shared__ float s_l[HG];
  __shared__ float s_mw[kWavesPerBlock][HG];
  __shared__ float s_f[kMaxSplits][HG];
  __shared__ float s_M[HG];
  __shared__ float s_L[HG];
  __shared__ float s_cur[HG];
  __shared__ int s_last;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int gi = lane / LPT, slice = lane % LPT;

  // ---- work item.  Consecutive workgroup ids land on different XCDs
  // (round robin over 8); remap so the splits of one head group share an XCD
  // and their partials stay in that XCD's L2 for the merge.
  const int units = a.num_layers * a.kv_heads * a.n_hgroups;
  const int64_t nblk = static_cast<int64_t>(units) * a.n_splits;
  int64_t g = blockIdx.x;
  if ((nblk & 7) == 0) g = (g & 7) * (nblk >> 3) + (g >> 3);
  const int unit = static_cast<int>(g / a.n_splits);
  const int split = static_cast<int>(g - static_cast<int64_t>(unit) * a.n_splits);
  const int lkv = unit / a.n_hgroups;
  const int hg = unit - lkv * a.n_hgroups;
  const int layer = lkv / a.kv_heads, kvh = lkv - layer * a.kv_heads;
  const int qh0 = kvh * a.group + hg * HG;

  // ---- tables, accumulators
  if constexpr (Fmt::kHasLut) {
    for (int e = tid; e < Fmt::kLutEntries; e += kBlock) {
      s_lut[0][e] = Fmt::lut_entry(e, a.cent_k);
      s_lut[1][e] = Fmt::lut_entry(e, a.cent_v);
    }
  }
  for (int o = tid; o < HG * D; o += kBlock) (&s_acc[0][0])[o] = 0.f;
  if (tid < HG) s_l[tid] = 0.f;

  // ---- queries: optional rotation (bit-identical to the reference), then
  // fold the softmax scale and log2(e) in.
  if (wave < HG) {
    float e[E];
    const int64_t qoff = (static_cast<int64_t>(layer) * a.query_heads + qh0 + wave) * D + lane * E;
    if (a.q_f16) {
      const __half* q = static_cast<const __half*>(a.q) + qoff;
#pragma unroll
      for (int i = 0; i < E; ++i) e[i] = __half2float(q[i]);
    } else {
      const float* q = static_cast<const float*>(a.q) + qoff;
#pragma unroll
      for (int i = 0; i < E; ++i) e[i] = q[i];
    }
    if (a.rotate_query) wave_rotate<D>(e, a.signs_right, a.signs_left, a.sqrt_d);
#pragma unroll
    for (int i = 0; i < E; ++i) s_q[wave][lane * E + i] = e[i] * a.q_scale;
  }
  __syncthreads();

  float qv[HG][SD];
#pragma unroll
  for (int h = 0; h < HG; ++h)
#pragma unroll
    for (int i = 0; i < SD; ++i) qv[h][i] = s_q[h][slice * SD + i];

  float m[HG], lsum[HG], acc[HG][SD];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    m[h] = -INFINITY;
    lsum[h] = 0.f;
#pragma unroll
    for (int i = 0; i < SD; ++i) acc[h][i] = 0.f;
  }

  // ---- main loop: wavefront `wave`, lane group `gi` takes tokens
  // t0 + wave*TPW + gi + k*TPB; one wavefront load covers TPW consecutive rows.
  const int64_t t0 = static_cast<int64_t>(split) * a.split_len;
  const int64_t t1 = min(a.seq_len, t0 + a.split_len);
  const uint8_t* kbase = a.k + static_cast<int64_t>(lkv) * a.cap * ROW;
  const uint8_t* vbase = a.v + static_cast<int64_t>(lkv) * a.cap * ROW;
  const typename Fmt::LutT* lut_k = s_lut[0];
  const typename Fmt::LutT* lut_v = s_lut[1];

  auto load_iter = [&](int64_t base, Raw (&kr)[U], Raw (&vr)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = base + u * TPB + gi;
      if (t < t1) {
        const int off = static_cast<int>(t * ROW);
        kr[u] = Fmt::load(kbase + off, slice);
        vr[u] = Fmt::load(vbase + off, slice);
      } else {
        kr[u] = Raw{};
        vr[u] = Raw{};
      }
    }
  };

  auto process = [&](const Raw& kr, const Raw& vr, bool valid) {
    float x[SD];
    Fmt::decode(kr, slice, lut_k, x);
    float s[HG];
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      float acc_s = 0.f;
#pragma unroll
      for (int i = 0; i < SD; ++i) acc_s = fmaf(qv[h][i], x[i], acc_s);
      s[h] = acc_s;
    }
#pragma unroll
    for (int mask = 1; mask < LPT; mask <<= 1)
#pragma unroll
      for (int h = 0; h < HG; ++h) s[h] += __shfl_xor(s[h], mask);
    float p[HG];
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      const float sv = valid ? s[h] : -INFINITY;
      if (sv > m[h] + kRescaleThreshold) {
        const float alpha = fast_exp2(m[h] - sv);
        lsum[h] *= alpha;
#pragma unroll
        for (int i = 0; i < SD; ++i) acc[h][i] *= alpha;
        m[h] = sv;
      }
      p[h] = valid ? fast_exp2(sv - m[h]) : 0.f;
      lsum[h] += p[h];
    }
    Fmt::decode(vr, slice, lut_v, x);
#pragma unroll
    for (int h = 0; h < HG; ++h)
#pragma unroll
      for (int i = 0; i < SD; ++i) acc[h][i] = fmaf(p[h], x[i], acc[h][i]);
  };

  {
    const int64_t first = t0 + wave * TPW;
    Raw kc[U], vc[U];
    load_iter(first, kc, vc);
    for (int64_t base = first; base < t1; base += U * TPB) {  // uniform per wavefront
      Raw kn[U], vn[U];
      load_iter(base + U * TPB, kn, vn);
#pragma unroll
      for (int u = 0; u < U; ++u) process(kc[u], vc[u], base + u * TPB + gi < t1);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        kc[u] = kn[u];
        vc[u] = vn[u];
      }
    }
  }

  // ---- combine the lane groups of this workgroup (log-sum-exp)
  float mw[HG];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    mw[h] = m[h];
#pragma unroll
    for (int mask = LPT; mask < kWave; mask <<= 1) mw[h] = fmaxf(mw[h], __shfl_xor(mw[h], mask));
  }
  if (lane == 0)
#pragma unroll
    for (int h = 0; h < HG; ++h) s_mw[wave][h] = mw[h];
  __syncthreads();
  float M[HG];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    M[h] = s_mw[0][h];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) M[h] = fmaxf(M[h], s_mw[w][h]);
    const float f = lsum[h] > 0.f ? fast_exp2(m[h] - M[h]) : 0.f;
#pragma unroll
    for (int i = 0; i < SD; ++i) atomicAdd(&s_acc[h][slice * SD + i], acc[h][i] * f);
    if (slice == 0) atomicAdd(&s_l[h], lsum[h] * f);
  }
  __syncthreads();

  const int64_t pidx = static_cast<int64_t>(unit) * a.n_splits + split;
  float* pacc = a.ws_acc + pidx * (HG * D);
  for (int o = tid; o < HG * D; o += kBlock) pacc[o] = (&s_acc[0][0])[o];
  if (tid < HG) a.ws_ml[pidx * HG + tid] = make_float2(M[tid], s_l[tid]);

  // ---- last workgroup of this head group merges all splits
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&a.counters[unit], 1u);
    s_last = (prev == static_cast<unsigned>(a.n_splits - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const int ns = a.n_splits;
  const float2* ml = a.ws_ml + static_cast<int64_t>(unit) * ns * HG;
  const float* accs = a.ws_acc + static_cast<int64_t>(unit) * ns * (HG * D);
  if (wave < HG) {
    const int h = wave;
    constexpr int PER = kMaxSplits / kWave;
    float2 v[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int s = lane + k * kWave;
      v[k] = s < ns ? ml[s * HG + h] : make_float2(-INFINITY, 0.f);
      mx = fmaxf(mx, v[k].x);
    }
#pragma unroll
    for (int mask = 1; mask < kWave; mask <<= 1) mx = fmaxf(mx, __shfl_xor(mx, mask));
    float lt = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int s = lane + k * kWave;
      const float f = v[k].y > 0.f ? fast_exp2(v[k].x - mx) : 0.f;
      if (s < ns) s_f[s][h] = f;
      lt += v[k].y * f;
    }
#pragma unroll
    for (int mask = 1; mask < kWave; mask <<= 1) lt += __shfl_xor(lt, mask);
    float sc = -INFINITY;
    if (a.cur_k != nullptr) {
      const float* ck = a.cur_k + static_cast<int64_t>(lkv) * D + lane * E;
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) dot = fmaf(s_q[h][lane * E + i], ck[i], dot);
#pragma unroll
      for (int mask = 1; mask < kWave; mask <<= 1) dot += __shfl_xor(dot, mask);
      sc = dot;
    }
    if (lane == 0) {
      s_M[h] = mx;
      s_L[h] = lt;
      s_cur[h] = sc;
    }
  }
  __syncthreads();

  for (int o = tid; o < HG * D; o += kBlock) {
    const int h = o / D, d = o - h * D;
    float A = 0.f;
#pragma unroll 16
    for (int s = 0; s < ns; ++s) A = fmaf(accs[static_cast<int64_t>(s) * (HG * D) + o], s_f[s][h], A);
    float L = s_L[h];
    if (a.cur_k != nullptr) {
      const float Mm = s_M[h], sc = s_cur[h];
      const float Mn = fmaxf(Mm, sc);
      const float f_old = L > 0.f ? fast_exp2(Mm - Mn) : 0.f;
      const float f_cur = fast_exp2(sc - Mn);
      A = A * f_old + a.cur_v[static_cast<int64_t>(lkv) * D + d] * f_cur;
      L = L * f_old + f_cur;
    }
    s_acc[h][d] = L > 0.f ? A / L : 0.f;
  }
  __syncthreads();

  if (wave < HG) {
    float e[E];
#pragma unroll
    for (int i = 0; i < E; ++i) e[i] = s_acc[wave][lane * E + i];
    if (a.inverse_output) wave_rotate<D>(e, a.signs_left, a.signs_right, a.sqrt_d);
    float* dst = a.out + (static_cast<int64_t>(layer) * a.query_heads + qh0 + wave) * D + lane * E;
#pragma unroll
    for (int i = 0; i < E; ++i) dst[i] = e[i];
  }
  if (tid == 0) a.counters[unit] = 0u;  // ready for the next call
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
#pragma unroll
  for (int mask = 1; mask < LPT; mask <<= 1) s += __shfl_xor(s, mask);
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
  for (int mask = 1; mask < kWave; mask <<= 1) mx = fmaxf(mx, __shfl_xor(mx, mask));
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int64_t t = tid; t < seq_len; t += kBlock) sum += expf(row[t] * scale - mx);
  for (int mask = 1; mask < kWave; mask <<= 1) sum += __shfl_xor(sum, mask);
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
  __shared__ float s_acc[D];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int gi = lane / LPT, slice = lane % LPT;
  const int b = blockIdx.x;
  for (int e = tid; e < Fmt::kLutEntries; e += kBlock) s_lut[e] = Fmt::lut_entry(e, cent);
  for (int d = tid; d < D; d += kBlock) s_acc[d] = 0.f;
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
  for (int i = 0; i < SD; ++i) atomicAdd(&s_acc[slice * SD + i], acc[i]);
  __syncthreads();
  for (int d = tid; d < D; d += kBlock) out[static_cast<int64_t>(b) * D + d] = s_acc[d];
}

// ============================================================== host helpers


int pick_hg(int group) {
  if (group % 4 == 0) return 4;
  if (group % 2 == 0) return 2;
  return 1;
}

struct Plan {
  int hg, n_hgroups, units, n_splits;
  int64_t split_len;
};

constexpr int kMinTokensPerSplit = 256;

int default_splits(int units, int64_t seq_len, int num_cus) {
  if (num_cus <= 0) num_cus = 256;
  const int64_t target = 2LL * num_cus;  // two workgroups per CU
  int64_t ns = (target + units - 1) / units;
  const int64_t by_len = std::max<int64_t>(1, (seq_len + kMinTokensPerSplit - 1) / kMinTokensPerSplit);
  ns = std::min(ns, by_len);
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

size_t workspace_bytes(int units, int hg, int head_dim, int n_splits) {
  const size_t counters = ((static_cast<size_t>(units) * sizeof(unsigned) + 255) / 256) * 256;
  const size_t ml = ((static_cast<size_t>(units) * n_splits * hg * sizeof(float2) + 255) / 256) * 256;
  const size_t acc = static_cast<size_t>(units) * n_splits * hg * head_dim * sizeof(float);
  return counters + ml + acc;
}

// Fills the split plan; tokens per split are a multiple of 256 rows so every
// split starts on a whole number of workgroup steps.
int make_plan(int num_layers, int kv_heads, int query_heads, int head_dim, int64_t seq_len, int n_splits, Plan* p) {
  if (num_layers <= 0 || kv_heads <= 0 || query_heads <= 0)
    return fail(TQ_ERR_BAD_ARG, "num_layers, kv_heads and query_heads must be positive");
  if (query_heads % kv_heads != 0)
    return fail(TQ_ERR_BAD_ARG, "query head count " + std::to_string(query_heads) + " must be divisible by kv_heads " +
                                    std::to_string(kv_heads));
  if (seq_len < 0) return fail(TQ_ERR_BAD_ARG, "seq_len must be non-negative");
  const int group = query_heads / kv_heads;
  p->hg = pick_hg(group);
  p->n_hgroups = group / p->hg;
  p->units = num_layers * kv_heads * p->n_hgroups;
  int ns = n_splits > 0 ? n_splits : default_splits(p->units, seq_len, device_cu_count());
  if (ns > kMaxSplits) return fail(TQ_ERR_BAD_ARG, "n_splits must be at most " + std::to_string(kMaxSplits));
  int64_t len = std::max<int64_t>(1, (seq_len + ns - 1) / ns);
  len = ((len + 255) / 256) * 256;
  const int64_t eff = std::max<int64_t>(1, (seq_len + len - 1) / len);
  p->n_splits = static_cast<int>(std::min<int64_t>(eff, ns));
  p->split_len = len;
  (void)head_dim;
  return TQ_OK;
}

template <class Fmt, int D, int HG>
void launch_decode(const DecodeArgs& a, int nblk, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL((decode_kernel<Fmt, D, HG>), dim3(nblk), dim3(kBlock), 0, stream, start, stop, 0, a);
  else
    hipLaunchKernelGGL((decode_kernel<Fmt, D, HG>), dim3(nblk), dim3(kBlock), 0, stream, a);
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
int decode_common(int fmt, const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                  int head_dim, const void* keys, const void* values, int64_t capacity, int64_t seq_len,
                  const float* cent_k, const float* cent_v, const float* signs_left, const float* signs_right,
                  int flags, const float* cur_k, const float* cur_v, int n_splits, void* workspace, float* out,
                  hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  int rc = check_geometry(head_dim, 0);
  if (rc) return rc;
  if (query == nullptr || out == nullptr || workspace == nullptr)
    return fail(TQ_ERR_BAD_ARG, "query, out and workspace must be non-null");
  if (query_dtype != TQ_F32 && query_dtype != TQ_F16) return fail(TQ_ERR_BAD_ARG, "query dtype must be F32 or F16");
  if (seq_len > 0 && (keys == nullptr || values == nullptr))
    return fail(TQ_ERR_BAD_ARG, "key and value slabs must be non-null");
  if (capacity < seq_len) return fail(TQ_ERR_BAD_ARG, "capacity must be >= seq_len");
  if ((cur_k == nullptr) != (cur_v == nullptr))
    return fail(TQ_ERR_BAD_ARG, "current_keys and current_values must both be given or both be null");
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
  rc = make_plan(num_layers, kv_heads, query_heads, head_dim, seq_len, n_splits, &p);
  if (rc) return rc;

  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const size_t counters = ((static_cast<size_t>(p.units) * sizeof(unsigned) + 255) / 256) * 256;
  const size_t ml = ((static_cast<size_t>(p.units) * p.n_splits * p.hg * sizeof(float2) + 255) / 256) * 256;

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
  a.n_splits = p.n_splits;
  a.split_len = p.split_len;
  a.counters = reinterpret_cast<unsigned*>(ws);
  a.ws_ml = reinterpret_cast<float2*>(ws + counters);
  a.ws_acc = reinterpret_cast<float*>(ws + counters + ml);
  a.out = out;
  const int nblk = p.units * p.n_splits;

  switch (fmt) {
    case 2:
      rc = dispatch_d<PackedB2>(a, head_dim, p.hg, nblk, stream, start, stop);
      break;
    case 3:
      rc = dispatch_d<PackedB3>(a, head_dim, p.hg, nblk, stream, start, stop);
      break;
    case 4:
      rc = dispatch_d<PackedB4>(a, head_dim, p.hg, nblk, stream, start, stop);
      break;
    case 16:
      rc = dispatch_d<DenseF16>(a, head_dim, p.hg, nblk, stream, start, stop);
      break;
    case 32:
      rc = dispatch_d<DenseF32>(a, head_dim, p.hg, nblk, stream, start, stop);
      break;
    default:
      return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(fmt));
  }
  if (rc) return rc;
  return launch_status("decode_kernel");
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

template <int D>
struct FwhtBody {
  static int run(const void* x, int x_dtype, float* y, int64_t rows, const float* s_first, const float* s_second,
                 hipStream_t stream) {
    const int64_t nblk = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
    const float sd = sqrt_f32(D);
    if (x_dtype == TQ_F16)
      hipLaunchKernelGGL((fwht_kernel<D, __half>), dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0, stream,
                         static_cast<const __half*>(x), y, rows, s_first, s_second, sd);
    else
      hipLaunchKernelGGL((fwht_kernel<D, float>), dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0, stream,
                         static_cast<const float*>(x), y, rows, s_first, s_second, sd);
    return launch_status("fwht_kernel");
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
};

template <int D, int BITS, typename T, bool DQ>
void launch_append(const AppendParams& p, hipStream_t stream) {
  const int64_t items = p.rows * p.streams;
  const int64_t nblk = (items + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL((append_kernel<D, BITS, T, DQ>), dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0, stream,
                     static_cast<const T*>(p.keys), static_cast<const T*>(p.values), p.rows, p.streams, p.seq_new,
                     p.rotate_keys, p.rotate_values, p.signs_left, p.signs_right, sqrt_f32(D), p.key_bnd,
                     p.value_bnd, p.key_cent, p.value_cent, p.key_codes, p.value_codes, p.capacity, p.offset,
                     p.key_out, p.value_out);
}

template <int D, int BITS>
void append_dtype(const AppendParams& p, hipStream_t stream) {
  if (p.dtype == TQ_F16) {
    if (p.dequant)
      launch_append<D, BITS, __half, true>(p, stream);
    else
      launch_append<D, BITS, __half, false>(p, stream);
  } else {
    if (p.dequant)
      launch_append<D, BITS, float, true>(p, stream);
    else
      launch_append<D, BITS, float, false>(p, stream);
  }
}

template <int D>
struct AppendBody {
  static int run(const AppendParams& p, int bits, hipStream_t stream) {
    switch (bits) {
      case 2:
        append_dtype<D, 2>(p, stream);
        break;
      case 3:
        append_dtype<D, 3>(p, stream);
        break;
      case 4:
        append_dtype<D, 4>(p, stream);
        break;
      default:
        return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
    }
    return launch_status("append_kernel");
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
  static int run(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, int bits,
                 const float* cent, float* out, hipStream_t stream) {
    const int64_t total = groups * seq_len * D;
    const int64_t nblk = (total + kBlock - 1) / kBlock;
    if (nblk == 0) return TQ_OK;
    switch (bits) {
      case 2:
        hipLaunchKernelGGL(unpack_kernel<2>, dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0, stream, codes, groups,
                           capacity, seq_len, D, cent, out);
        break;
      case 3:
        hipLaunchKernelGGL(unpack_kernel<3>, dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0, stream, codes, groups,
                           capacity, seq_len, D, cent, out);
        break;
      case 4:
        hipLaunchKernelGGL(unpack_kernel<4>, dim3(static_cast<unsigned>(nblk)), dim3(kBlock), 0, stream, codes, groups,
                           capacity, seq_len, D, cent, out);
        break;
      default:
        return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
    }
    return launch_status("unpack_kernel");
  }
};

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
  return with_d<AppendBody>(head_dim, p, bits, stream);
}

int tq_quantize_dequantize(const void* keys, const void* values, int dtype, int64_t rows, int head_dim, int bits,
                           const float* signs_left, const float* signs_right, int flags,
                           const float* key_boundaries, const float* value_boundaries,
                           const float* key_centroids, const float* value_centroids, float* key_out,
                           float* value_out, hipStream_t stream) {
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
  return with_d<AppendBody>(head_dim, p, bits, stream);
}

int tq_unpack_dequantize(const uint32_t* codes, int64_t groups, int64_t capacity, int64_t seq_len, int head_dim,
                         int bits, const float* centroids, float* out, hipStream_t stream) {
  int rc = check_geometry(head_dim, bits);
  if (rc) return rc;
  if (groups < 0 || seq_len < 0 || capacity < seq_len) return fail(TQ_ERR_BAD_ARG, "bad unpack extents");
  if (groups == 0 || seq_len == 0) return TQ_OK;
  if (!codes || !centroids || !out) return fail(TQ_ERR_BAD_ARG, "null pointer argument");
  return with_d<UnpackBody>(head_dim, codes, groups, capacity, seq_len, bits, centroids, out, stream);
}

int tq_decode_default_splits(int num_layers, int kv_heads, int query_heads, int head_dim, int64_t seq_len,
                             int num_cus) {
  if (num_layers <= 0 || kv_heads <= 0 || query_heads <= 0 || query_heads % kv_heads != 0)
    return fail(TQ_ERR_BAD_ARG, "bad head configuration");
  (void)head_dim;
  const int group = query_heads / kv_heads;
  const int hg = pick_hg(group);
  const int units = num_layers * kv_heads * (group / hg);
  return default_splits(units, seq_len, num_cus);
}

size_t tq_decode_workspace_bytes(int num_layers, int kv_heads, int query_heads, int head_dim, int n_splits,
                                 int num_cus) {
  if (num_layers <= 0 || kv_heads <= 0 || query_heads <= 0 || query_heads % kv_heads != 0) return 0;
  const int group = query_heads / kv_heads;
  const int hg = pick_hg(group);
  const int units = num_layers * kv_heads * (group / hg);
  int ns = n_splits;
  if (ns <= 0) ns = default_splits(units, static_cast<int64_t>(kMaxSplits) * kMinTokensPerSplit, num_cus);
  ns = std::min(ns, kMaxSplits);
  return workspace_bytes(units, hg, head_dim, ns);
}

int tq_decode(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads, int head_dim,
              int bits, const uint32_t* key_codes, const uint32_t* value_codes, int64_t capacity, int64_t seq_len,
              const float* key_centroids, const float* value_centroids, const float* signs_left,
              const float* signs_right, int flags, const float* current_keys, const float* current_values,
              int n_splits, void* workspace, float* out, hipStream_t stream) {
  return tq_decode_timed(query, query_dtype, num_layers, query_heads, kv_heads, head_dim, bits, key_codes,
                         value_codes, capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right,
                         flags, current_keys, current_values, n_splits, workspace, out, stream, nullptr, nullptr);
}

int tq_decode_timed(const void* query, int query_dtype, int num_layers, int query_heads, int kv_heads,
                    int head_dim, int bits, const uint32_t* key_codes, const uint32_t* value_codes,
                    int64_t capacity, int64_t seq_len, const float* key_centroids, const float* value_centroids,
                    const float* signs_left, const float* signs_right, int flags, const float* current_keys,
                    const float* current_values, int n_splits, void* workspace, float* out, hipStream_t stream,
                    hipEvent_t start, hipEvent_t stop) {
  if (!valid_bits(bits)) return fail(TQ_ERR_UNSUPPORTED, "Unsupported bit width: " + std::to_string(bits));
  return decode_common(bits, query, query_dtype, num_layers, query_heads, kv_heads, head_dim, key_codes,
                       value_codes, capacity, seq_len, key_centroids, value_centroids, signs_left, signs_right, flags,
                       current_keys, current_values, n_splits, workspace, out, stream, start, stop);
}

int tq_decode_dense(const void* query, int query_dtype, const void* keys, const void* values, int kv_dtype,
                    int num_layers, int query_heads, int kv_heads, int head_dim, int64_t capacity, int64_t seq_len,
                    const float* signs_left, const float* signs_right, int flags, int n_splits, void* workspace,
                    float* out, hipStream_t stream) {
  return tq_decode_dense_timed(query, query_dtype, keys, values, kv_dtype, num_layers, query_heads, kv_heads,
                               head_dim, capacity, seq_len, signs_left, signs_right, flags, n_splits, workspace, out,
                               stream, nullptr, nullptr);
}

int tq_decode_dense_timed(const void* query, int query_dtype, const void* keys, const void* values, int kv_dtype,
                          int num_layers, int query_heads, int kv_heads, int head_dim, int64_t capacity,
                          int64_t seq_len, const float* signs_left, const float* signs_right, int flags,
                          int n_splits, void* workspace, float* out, hipStream_t stream, hipEvent_t start,
                          hipEvent_t stop) {
  if (kv_dtype != TQ_F16 && kv_dtype != TQ_F32) return fail(TQ_ERR_BAD_ARG, "kv dtype must be F32 or F16");
  return decode_common(kv_dtype == TQ_F16 ? 16 : 32, query, query_dtype, num_layers, query_heads, kv_heads, head_dim,
                       keys, values, capacity, seq_len, nullptr, nullptr, signs_left, signs_right, flags, nullptr,
                       nullptr, n_splits, workspace, out, stream, start, stop);
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

}  // extern "C"
