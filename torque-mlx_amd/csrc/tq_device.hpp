// Device-side building blocks for the packed rotated KV-cache kernels (gfx950).
//
// Wavefront = 64 lanes.  A D-vector held by one wavefront is split so that
// lane l owns elements [l*E, l*E + E), E = D / 64.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tq {

constexpr int kWave = 64;
constexpr int kBlock = 256;  // 4 wavefronts per workgroup
constexpr int kWavesPerBlock = kBlock / kWave;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float to_f32<__half>(__half v) {
  return __half2float(v);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier that publishes LDS writes only: it waits for the
// wavefront's LDS operations (lgkmcnt) and not for its outstanding global
// loads.  __syncthreads() fences global memory as well, which waits for every
// load in flight (vmcnt counts loads), so a barrier placed after a row
// prefetch would hold each wavefront until its prefetched rows had landed.
// Use it only where the wavefronts exchange data through LDS alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------
// Cross-lane data movement without LDS.
//
// DPP moves inside 16-lane rows.  Every control used here has a valid source
// lane for every lane, so bound_ctrl changes nothing but lets the compiler
// fold the move into the consuming VALU instruction.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;       // lane i <-> 15 - i within 16
constexpr int kDppRor4 = 0x124;         // lane i <- lane (i - 4) mod 16 (rotate right: data moves up)
constexpr int kDppRor8 = 0x128;         // lane i <- lane (i + 8) mod 16, i.e. i xor 8
constexpr int kDppRor12 = 0x12C;        // lane i <- lane (i + 4) mod 16

// gfx950 v_permlane16_swap / v_permlane32_swap.  With x in the first operand
// and y in the second, for every lane pair (i, i xor M), M = 16 or 32, i the
// lower lane: afterwards first = (x_i, y_i) and second = (x_(i^M), y_(i^M)),
// listing (lower lane, upper lane).  So first + second gives the lower lane
// x_i + x_(i^M) and the upper lane y_i + y_(i^M): one reduce-scatter step;
// with x = y it is an all-reduce step.
struct LanePair {
  float first, second;
};
template <int M>
__device__ __forceinline__ LanePair permlane_swap(float x, float y) {
  static_assert(M == 16 || M == 32, "permlane swaps pair lanes 16 or 32 apart");
  const unsigned ux = __builtin_bit_cast(unsigned, x), uy = __builtin_bit_cast(unsigned, y);
  if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(ux, uy, false, false);
    return {__builtin_bit_cast(float, static_cast<unsigned>(r[0])), __builtin_bit_cast(float, static_cast<unsigned>(r[1]))};
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(ux, uy, false, false);
    return {__builtin_bit_cast(float, static_cast<unsigned>(r[0])), __builtin_bit_cast(float, static_cast<unsigned>(r[1]))};
  }
}

struct OpSum {
  __device__ static float f(float a, float b) { return a + b; }
};
struct OpMax {
  __device__ static float f(float a, float b) { return fmaxf(a, b); }
};

// All-reduce over the lane pairs (i, i xor M), M = 16 or 32.
template <int M, class Op>
__device__ __forceinline__ float xor_reduce(float v) {
  const LanePair r = permlane_swap<M>(v, v);
  return Op::f(r.first, r.second);
}

// Reduction over aligned groups of N consecutive lanes (N a power of two up
// to 64); every lane of a group receives the group result.  After the two
// quad steps each quad holds its result; the mirror steps then pair a quad
// (half row) with the other quad (half row) of the same 8 (16) lanes.
template <int N, class Op = OpSum>
__device__ __forceinline__ float group_reduce(float v) {
  if constexpr (N >= 2) v = Op::f(v, dpp_move<kDppXor1>(v));
  if constexpr (N >= 4) v = Op::f(v, dpp_move<kDppXor2>(v));
  if constexpr (N >= 8) v = Op::f(v, dpp_move<kDppHalfMirror>(v));
  if constexpr (N >= 16) v = Op::f(v, dpp_move<kDppMirror>(v));
  if constexpr (N >= 32) v = xor_reduce<16, Op>(v);
  if constexpr (N >= 64) v = xor_reduce<32, Op>(v);
  return v;
}
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  return group_reduce<N, OpSum>(v);
}

// Quad rotations: every lane of a quad reads the lane R positions back
// (quad_rotate_from) or ahead (quad_rotate_to), positions taken mod 4.
template <int R>
__device__ __forceinline__ float quad_rotate_from(float v) {
  constexpr int c = ((0 - R) & 3) | (((1 - R) & 3) << 2) | (((2 - R) & 3) << 4) | (((3 - R) & 3) << 6);
  return dpp_move<c>(v);
}
template <int R>
__device__ __forceinline__ float quad_rotate_to_t(float v) {
  constexpr int c = (R & 3) | (((1 + R) & 3) << 2) | (((2 + R) & 3) << 4) | (((3 + R) & 3) << 6);
  return dpp_move<c>(v);
}
__device__ __forceinline__ float quad_rotate_to(float v, int r) {
  switch (r & 3) {
    case 0:
      return v;
    case 1:
      return quad_rotate_to_t<1>(v);
    case 2:
      return quad_rotate_to_t<2>(v);
    default:
      return quad_rotate_to_t<3>(v);
  }
}

// Value of quad position S, broadcast to every lane of each quad.
template <int S>
__device__ __forceinline__ float quad_broadcast_t(float v) {
  return dpp_move<S | (S << 2) | (S << 4) | (S << 6)>(v);
}
__device__ __forceinline__ float quad_broadcast(float v, int s) {
  switch (s) {
    case 0:
      return quad_broadcast_t<0>(v);
    case 1:
      return quad_broadcast_t<1>(v);
    case 2:
      return quad_broadcast_t<2>(v);
    default:
      return quad_broadcast_t<3>(v);
  }
}

// Sum of the quads of an aligned group of N lanes (N a power of two, 4..64)
// in which quad position p of one quad is matched with position 3 - p of the
// neighbouring quad (row_half_mirror, row_mirror) and with the same position
// in the other half rows (lanes 16 and 32 apart).
template <int N>
__device__ __forceinline__ float cross_quad_sum(float v) {
  if constexpr (N >= 8) v += dpp_move<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp_move<kDppMirror>(v);
  if constexpr (N >= 32) v = xor_reduce<16, OpSum>(v);
  if constexpr (N >= 64) v = xor_reduce<32, OpSum>(v);
  return v;
}

// Reduction over the lanes of a wavefront that share (lane mod G), G a power
// of two >= 4; every lane receives the result of its residue class.  Inside a
// 16-lane row the class is closed under rotation by 4 and 8, so two rotate
// steps cover it; the permlane steps join the rows.
template <int G, class Op>
__device__ __forceinline__ float strided_reduce(float v) {
  static_assert(G >= 4 && G <= kWave && (G & (G - 1)) == 0, "stride must be a power of two in [4, 64]");
  if constexpr (G <= 4) v = Op::f(v, dpp_move<kDppRor4>(v));
  if constexpr (G <= 8) v = Op::f(v, dpp_move<kDppRor8>(v));
  if constexpr (G <= 16) v = xor_reduce<16, Op>(v);
  if constexpr (G <= 32) v = xor_reduce<32, Op>(v);
  return v;
}

// The value of lane (lane xor M), M a power of two below 64, moved by DPP
// inside rows and by the permlane swaps across them.  Exact data movement.
template <int M>
__device__ __forceinline__ float xor_partner(float v, int lane) {
  if constexpr (M == 1) {
    return dpp_move<kDppXor1>(v);
  } else if constexpr (M == 2) {
    return dpp_move<kDppXor2>(v);
  } else if constexpr (M == 4) {
    return dpp_move<0x1B>(dpp_move<kDppHalfMirror>(v));  // 7 - i, then quad reversal: i xor 4
  } else if constexpr (M == 8) {
    return dpp_move<kDppRor8>(v);
  } else {
    const LanePair r = permlane_swap<M>(v, v);
    return (lane & M) ? r.first : r.second;
  }
}

// ---------------------------------------------------------------------------
// Walsh-Hadamard transform of one D-vector held by a wavefront.
//
// Butterfly order and operands are those of the reference's float32 numpy
// transform (rotation.py:19-32): steps 1, 2, 4, ..., each producing
// (left + right, left - right) with `left` the lower index.  Every element
// sees the same sequence of IEEE float32 adds/subtracts with the same
// operands, so the result is bit-identical to the reference.
// One cross-lane butterfly stage: partners lane and lane xor M.
template <int M, int E>
__device__ __forceinline__ void fwht_cross(float (&v)[E], int lane) {
  const bool upper = (lane & M) != 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float other = xor_partner<M>(v[i], lane);
    v[i] = upper ? __fsub_rn(other, v[i]) : __fadd_rn(v[i], other);
  }
}

// The stages 16 and 32 apart on two of a lane's elements at once: after one
// permlane swap of (a, b) the lower lane of each pair holds (a_lower,
// a_upper) and the upper lane (b_lower, b_upper), so one add and one subtract
// form both butterflies (left + right, left - right, left the lower lane, as
// in fwht_cross), and a second swap of (sum, difference) returns new a and
// new b to their lanes.  Same operations on the same operands: bit-identical.
template <int M, int E>
__device__ __forceinline__ void fwht_cross_pairs(float (&v)[E]) {
  static_assert(E % 2 == 0, "pairs of elements");
#pragma unroll
  for (int i = 0; i < E; i += 2) {
    const LanePair p = permlane_swap<M>(v[i], v[i + 1]);
    const LanePair q = permlane_swap<M>(__fadd_rn(p.first, p.second), __fsub_rn(p.first, p.second));
    v[i] = q.first;
    v[i + 1] = q.second;
  }
}

template <int D>
__device__ __forceinline__ void wave_fwht(float (&v)[D / kWave]) {
  constexpr int E = D / kWave;
  const int lane = lane_id();
#pragma unroll
  for (int s = 1; s < E; s <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if ((i & s) == 0) {
        const float a = v[i], b = v[i + s];
        v[i] = __fadd_rn(a, b);
        v[i + s] = __fsub_rn(a, b);
      }
    }
  }
  fwht_cross<1>(v, lane);
  fwht_cross<2>(v, lane);
  fwht_cross<4>(v, lane);
  fwht_cross<8>(v, lane);
  if constexpr (E >= 2) {
    fwht_cross_pairs<16>(v);
    fwht_cross_pairs<32>(v);
  } else {
    fwht_cross<16>(v, lane);
    fwht_cross<32>(v, lane);
  }
}

// y = s_second * (H (s_first * x)) / sqrt(D), with the reference's operation
// order (rotation.py:88-102): multiply by the first signs, transform, divide
// by float32(sqrt(D)) (correctly rounded), multiply by the second signs.
// apply():   s_first = signs_right, s_second = signs_left
// inverse(): s_first = signs_left,  s_second = signs_right
// wave_rotate_signs takes this lane's E signs of each vector in registers;
// wave_rotate loads them.
template <int D>
__device__ __forceinline__ void wave_rotate_signs(float (&v)[D / kWave], const float (&s_first)[D / kWave],
                                                  const float (&s_second)[D / kWave], float sqrt_d) {
  constexpr int E = D / kWave;
#pragma unroll
  for (int i = 0; i < E; ++i) v[i] = __fmul_rn(v[i], s_first[i]);
  wave_fwht<D>(v);
  if constexpr (D == 64 || D == 256) {
    // sqrt(D) is a power of two (sqrt_d = 8 or 16 exactly): multiplying by
    // its exact reciprocal rounds like the division, denormals included
    constexpr float kInv = D == 64 ? 0.125f : 0.0625f;
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = __fmul_rn(__fmul_rn(v[i], kInv), s_second[i]);
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = __fmul_rn(__fdiv_rn(v[i], sqrt_d), s_second[i]);
  }
}
template <int D>
__device__ __forceinline__ void wave_rotate(float (&v)[D / kWave], const float* __restrict__ s_first,
                                            const float* __restrict__ s_second, float sqrt_d) {
  constexpr int E = D / kWave;
  const int base = lane_id() * E;
  float f[E], g[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    f[i] = s_first[base + i];
    g[i] = s_second[base + i];
  }
  wave_rotate_signs<D>(v, f, g, sqrt_d);
}

// ---------------------------------------------------------------------------
// Quantizer: code = number of boundaries strictly below x (quantization.py:139-148,
// mlx_ops.py:271-273).  Ties go to the lower code; NaN gives 0.
template <int BITS>
__device__ __forceinline__ uint32_t quantize_count(float x, const float* __restrict__ bnd) {
  uint32_t c = 0;
#pragma unroll
  for (int k = 0; k < (1 << BITS) - 1; ++k) c += (x > bnd[k]) ? 1u : 0u;
  return c;
}

// Packed word `w` of a row whose codes sit in `codes[0..D)`: LSB-first
// bitstream, code j at bit j*BITS, the high bits of a code that crosses a word
// boundary continue at bit 0 of the next word (quantization.py:156-173).
template <int BITS, int D>
__device__ __forceinline__ uint32_t pack_word(const uint8_t* codes, int w) {
  const int bit0 = 32 * w;
  const int j0 = bit0 / BITS;
  int j1 = (bit0 + 31) / BITS;
  if (j1 > D - 1) j1 = D - 1;
  uint32_t word = 0;
  for (int j = j0; j <= j1; ++j) {
    const int o = j * BITS - bit0;
    const uint32_t c = codes[j];
    word |= (o >= 0) ? (c << o) : (c >> (-o));
  }
  return word;
}

// Code j of a packed row (straddle-aware), for the unpack kernels.
template <int BITS>
__device__ __forceinline__ uint32_t unpack_code(const uint32_t* __restrict__ row, int j) {
  const int bit = j * BITS;
  const int w = bit >> 5, s = bit & 31;
  uint32_t v = row[w] >> s;
  if (s + BITS > 32) v |= row[w + 1] << (32 - s);
  return v & ((1u << BITS) - 1u);
}

// ---------------------------------------------------------------------------
// Lane-slice formats for the decode kernels.  A token row is split into
// D / kSliceDims slices; one lane owns one slice of one token.  `load` reads
// the slice's raw bits from the row, `decode` turns them into kSliceDims
// float32 values using an LDS lookup table built from the centroids.

// ---- raw buffer loads.  A buffer resource bounds what a loop may read:
// a load whose bytes lie past num_records returns zeros and touches no
// memory, so rows past the end of a range need no clamp.  Untyped loads on
// this target take DATA_FORMAT = 32 bits in the descriptor's last word.
constexpr int kBufferWord3 = 0x00020000;
// Cache policy of the K/V row loads: nontemporal (the `nt` bit).  A decode
// reads every row once per call, so the rows should not displace what stays
// cached between launches (the per-split partials the merge kernel reads
// next): measured at M, 16.5 -> 15.7 us per step with the same split-kernel
// time; at C4 30.8 -> 29.7.
constexpr int kRowLoadPolicy = 2;
using BufferRsrc = __amdgpu_buffer_rsrc_t;
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ BufferRsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferWord3);
}

// 4-bit: 16 dims = 8 bytes = words 2s, 2s+1; one table entry per byte holds
// the centroids of its low and high nibble.
struct PackedB4 {
  static constexpr int kBits = 4;
  static constexpr int kSliceDims = 16;
  static constexpr bool kHasLut = true;
  static constexpr int kLutEntries = 256;
  using LutT = float2;
  struct Raw {
    uint32_t a, b;
  };
  template <int D>
  static constexpr int row_bytes() {
    return D * kBits / 8;
  }
  __device__ static LutT lut_entry(int e, const float* __restrict__ c) { return make_float2(c[e & 15], c[e >> 4]); }
  __device__ static float first_centroid(const LutT& t) { return t.x; }
  __device__ static Raw load(const uint8_t* __restrict__ row, int slice) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + 8 * slice);
    return {v.x, v.y};
  }
  __device__ static int slice_offset(int slice) { return 8 * slice; }
  __device__ static Raw load(BufferRsrc r, int off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kRowLoadPolicy);
    return {v.x, v.y};
  }
  __device__ static void decode(const Raw& r, int /*slice*/, const LutT* __restrict__ lut, float (&x)[kSliceDims]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t word = (j < 4) ? r.a : r.b;
      const uint32_t byte = (word >> (8 * (j & 3))) & 0xffu;
      const float2 c = lut[byte];
      x[2 * j] = c.x;
      x[2 * j + 1] = c.y;
    }
  }
};

// 2-bit: 16 dims = 1 word; one table entry per byte holds 4 centroids.
struct PackedB2 {
  static constexpr int kBits = 2;
  static constexpr int kSliceDims = 16;
  static constexpr bool kHasLut = true;
  static constexpr int kLutEntries = 256;
  using LutT = float4;
  struct Raw {
    uint32_t a;
  };
  template <int D>
  static constexpr int row_bytes() {
    return D * kBits / 8;
  }
  __device__ static LutT lut_entry(int e, const float* __restrict__ c) {
    return make_float4(c[e & 3], c[(e >> 2) & 3], c[(e >> 4) & 3], c[(e >> 6) & 3]);
  }
  __device__ static float first_centroid(const LutT& t) { return t.x; }
  __device__ static Raw load(const uint8_t* __restrict__ row, int slice) {
    return {*reinterpret_cast<const uint32_t*>(row + 4 * slice)};
  }
  __device__ static int slice_offset(int slice) { return 4 * slice; }
  __device__ static Raw load(BufferRsrc r, int off) { return {__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kRowLoadPolicy)}; }
  __device__ static void decode(const Raw& r, int /*slice*/, const LutT* __restrict__ lut, float (&x)[kSliceDims]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 c = lut[(r.a >> (8 * j)) & 0xffu];
      x[4 * j] = c.x;
      x[4 * j + 1] = c.y;
      x[4 * j + 2] = c.z;
      x[4 * j + 3] = c.w;
    }
  }
};

// 3-bit: 16 dims = 48 bits starting at bit 48*s, i.e. words (3s)>>1 and the
// next one, shifted right by 16 for odd slices.  Codes straddle word
// boundaries; one table entry per 6-bit code pair holds both centroids.
struct PackedB3 {
  static constexpr int kBits = 3;
  static constexpr int kSliceDims = 16;
  static constexpr bool kHasLut = true;
  static constexpr int kLutEntries = 64;
  using LutT = float2;
  struct Raw {
    uint32_t a, b;
  };
  template <int D>
  static constexpr int row_bytes() {
    return D * kBits / 8;
  }
  __device__ static LutT lut_entry(int e, const float* __restrict__ c) { return make_float2(c[e & 7], c[e >> 3]); }
  __device__ static float first_centroid(const LutT& t) { return t.x; }
  __device__ static Raw load(const uint8_t* __restrict__ row, int slice) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(row) + ((3 * slice) >> 1);
    return {w[0], w[1]};
  }
  __device__ static int slice_offset(int slice) { return 4 * ((3 * slice) >> 1); }
  __device__ static Raw load(BufferRsrc r, int off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kRowLoadPolicy);
    return {v.x, v.y};
  }
  __device__ static void decode(const Raw& r, int slice, const LutT* __restrict__ lut, float (&x)[kSliceDims]) {
    const uint64_t z = ((static_cast<uint64_t>(r.b) << 32) | r.a) >> ((slice & 1) * 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float2 c = lut[static_cast<uint32_t>(z >> (6 * j)) & 63u];
      x[2 * j] = c.x;
      x[2 * j + 1] = c.y;
    }
  }
};

// Dense float16 rows: 8 dims = 16 bytes per slice.
struct DenseF16 {
  static constexpr int kBits = 0;  // not a packed format
  static constexpr int kSliceDims = 8;
  static constexpr bool kHasLut = false;
  static constexpr int kLutEntries = 1;
  using LutT = float;
  struct Raw {
    uint4 v;
  };
  template <int D>
  static constexpr int row_bytes() {
    return D * 2;
  }
  __device__ static LutT lut_entry(int, const float*) { return 0.f; }
  __device__ static float first_centroid(const LutT& t) { return t; }
  __device__ static Raw load(const uint8_t* __restrict__ row, int slice) {
    return {*reinterpret_cast<const uint4*>(row + 16 * slice)};
  }
  __device__ static int slice_offset(int slice) { return 16 * slice; }
  __device__ static Raw load(BufferRsrc r, int off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kRowLoadPolicy);
    return {make_uint4(v.x, v.y, v.z, v.w)};
  }
  __device__ static void decode(const Raw& r, int, const LutT*, float (&x)[kSliceDims]) {
    const uint32_t w[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[j] & 0xffffu)));
      x[2 * j + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[j] >> 16)));
    }
  }
};

// Dense float32 rows: 4 dims = 16 bytes per slice.
struct DenseF32 {
  static constexpr int kBits = 0;  // not a packed format
  static constexpr int kSliceDims = 4;
  static constexpr bool kHasLut = false;
  static constexpr int kLutEntries = 1;
  using LutT = float;
  struct Raw {
    float4 v;
  };
  template <int D>
  static constexpr int row_bytes() {
    return D * 4;
  }
  __device__ static LutT lut_entry(int, const float*) { return 0.f; }
  __device__ static float first_centroid(const LutT& t) { return t; }
  __device__ static Raw load(const uint8_t* __restrict__ row, int slice) {
    return {*reinterpret_cast<const float4*>(row + 16 * slice)};
  }
  __device__ static int slice_offset(int slice) { return 16 * slice; }
  __device__ static Raw load(BufferRsrc r, int off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kRowLoadPolicy);
    return {make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w))};
  }
  __device__ static void decode(const Raw& r, int, const LutT*, float (&x)[kSliceDims]) {
    x[0] = r.v.x;
    x[1] = r.v.y;
    x[2] = r.v.z;
    x[3] = r.v.w;
  }
};

}  // namespace tq
