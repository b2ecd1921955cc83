// decode_mx_kernel -- split-K packed decode for groups of 4 query heads on the
// gfx950 matrix cores with 16x16x32 float16 products (v_mfma_f32_16x16x32_f16).
//
// Included by torque_hip.hip (uses DecodeArgs, finish_row and tq_device.hpp).
//
// Arithmetic.  Every product is formed from exact float16 splits and summed in
// float32: a centroid c is stored as hi = f16(c) and lo = f16(c - hi) (so
// |c - hi - lo| <= 2^-22 |c|), the scaled query q likewise, and a softmax
// weight p as hi = p with its low 13 mantissa bits cleared (exact in f16) and
// lo = f16(p - hi).  The products hi*hi, hi*lo, lo*hi, lo*lo are exact in
// float32, so a score or value term carries at most ~2^-21 relative error
// against the float32 product (2^-24), and every sum is a float32 sum.
// Before splitting, the centroids, the query and the weights are scaled by
// powers of two (exact) so that their largest magnitude sits in
// [2^14, 2^15): no f16 overflow, and the lo parts stay clear of f16
// subnormals for all but negligible terms.  The scales are undone with one
// exact multiply per score and per output.  Per-vector scales (the scaled
// decode) are not taken here: they would multiply the weights, whose split
// has no headroom for a factor of unknown size; that decode runs on the
// float32 split kernel.
//
// Lane layouts (wave of 64 lanes; n = lane % 16, g = lane / 16; checked on the
// device: the A operand of lane l supplies row l % 16, the B operand column
// l % 16, both with the 8 k-slots of lane group g, and the 16x16 result holds
// column l % 16, rows 4g .. 4g + 3 in its 4 registers).
//
//   A wave takes 16 consecutive rows (tokens) per iteration: token 4g + r is
//   row r of lane group g's part of every result tile.
//
//   Scores, S[token][col] += K[token][k] * Q[k][col]: A = key rows, lane
//   (n, g) holding token n and the g-th quarter of its packed row (a 128-bit
//   load at D = 128); each key byte (two codes, dims 2i, 2i + 1) is one lookup
//   in a table of (hi pair, lo pair) and fills k-slots (hi(d), hi(d+1),
//   lo(d), lo(d+1)), so one 16x16x32 product covers 4 dims per lane group.
//   B = the query: column h holds the hi split of head h's query, column
//   4 + h its lo split, columns 8..15 zero; each query value appears in the
//   k-slots of both the hi and the lo key part.  The score of head h is
//   column h + column 4 + h (a row_ror:12 DPP add: lane i reads lane i + 4 of
//   its row), so lanes n < 4 end up with
//   head n's scores of their 4 tokens.
//
//   Softmax: the four score registers are spread over the 16 lanes of a
//   row (DPP moves), so that lane m holds head m % 4's score of token
//   4g + m / 4 % 4 and every exp2 is a useful one.
//
//   Values, O[row][dim] += P[row][k] * V[k][dim]: B = value codes, lane
//   (n, g) reading dword n (8 dims) of rows 4g .. 4g + 3; the nibbles of a
//   dim in two tokens are interleaved into one byte, whose lookup in the
//   value table gives (hi(t), lo(t)) and (hi(t'), lo(t')), so the k-slots are
//   4 tokens x (hi, lo).  A = weights: row h holds the hi split of head h's
//   weights, row 4 + h the lo split, each weight as the pair (w, w) facing a
//   token's (hi, lo) k-slots (gathered from the softmax lanes by DPP moves).
//   One product covers 16 tokens x 16 dims; the output of head h is row h +
//   row 4 + h (lane groups 0 and 1, one permlane16 swap at the end).
//
// Tables: 256 entries x 8 bytes per stream, each entry replicated 32 times
// so that lane l reads copy l % 32: entry e, copy c at byte e * 256 + c * 8
// (64 KB per stream), which keeps 32 lanes' 8-byte reads on 32 distinct bank
// pairs whatever the codes (measured: 2.96 cycles per wave read against 6.6
// for one shared 2 KB table).  The key table sits at LDS byte 0, the value
// table at 65536, so a lookup address is one v_perm_b32 that puts the code
// byte in bits 8..15 of the lane's base.  Wavefronts 4..11 write the tables
// straight from the 32 centroids (held one per lane) while wavefronts 0..3
// prepare the queries; one barrier ends the set-up.

namespace mx {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

// Wavefronts per workgroup (one workgroup per compute unit): 12, three per
// SIMD, at head_dim 64 / 128; 8, two per SIMD with up to 256 VGPRs each, at
// head_dim 256, whose accumulators and query operands take twice the
// registers.
template <int D>
constexpr int waves_of() {
  return D == 256 ? 8 : 12;
}
template <int D>
constexpr int threads_of() {
  return waves_of<D>() * kWave;
}
constexpr int kTile = 16;                 // tokens per wavefront iteration
constexpr int kTilesPerBlock = 8;
constexpr int kStride = kTilesPerBlock * kTile;  // rows per block (the unit dealt out to the splits)
constexpr int kCopies = 32;               // lane-private copies of a table entry
constexpr int kTableBytes = 256 * kCopies * 8;
constexpr int kPrefetch = 2;              // tiles whose loads are in flight ahead

// LDS: the two tables, reused for the cross-wavefront reduction after the loop.
template <int D>
struct Smem {
  static constexpr int kQbStride = D + 8;                // f16 elements per padded row (16-byte skew per row)
  static constexpr int kQbBytes = 8 * kQbStride * 2;     // f16 query splits [8 cols][D]
  static constexpr int kQBytes = 4 * D * 4;           // float32 scaled query [4][D]
  static constexpr int kCurBytes = 2 * D * 4 + 2 * D;  // append mode: s_cur [2][D] + codes [2][D]
  static constexpr int kMisc = 1024;
  static constexpr int kNW = waves_of<D>();
  static constexpr int kRS = D == 128 ? D + 6 : D < 128 ? D + 10 : D + 18;  // padded reduction row (floats)
  static constexpr int kRedBytes = kNW * 4 * kRS * 4 + 2 * kNW * 4 * 4;      // rows, then (max, sum) per wave
  static constexpr int kQb = 2 * kTableBytes;
  static constexpr int kQ = kQb + kQbBytes;
  static constexpr int kCur = kQ + kQBytes;
  static constexpr int kMiscOff = kCur + kCurBytes;
  static constexpr int kSetup = kMiscOff + kMisc;
  // The reduction sits beside the tables where the LDS holds both (head_dim
  // 64 and 128), so each wavefront deposits its partial as soon as its own
  // loop ends; at head_dim 256 it reuses the table area after a barrier.
  static constexpr bool kRedApart = kSetup + kRedBytes <= 160 * 1024;
  static constexpr int kRed = kRedApart ? kSetup : 0;
  static constexpr int kTotal = kRedApart ? kSetup + kRedBytes : kSetup;
  static_assert(kRedApart || kRedBytes <= 2 * kTableBytes, "reduction fits in the table area");
};

__device__ __forceinline__ uint32_t pack_f16x2(_Float16 lo, _Float16 hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
}

// Largest magnitude of x[0..n) -> exponent shift that maps it into [2^14, 2^15).
__device__ __forceinline__ int scale_shift(float maxabs) {
  if (!(maxabs > 0.f) || !isfinite(maxabs)) return 0;
  int e;
  frexpf(maxabs, &e);  // maxabs = m 2^e, m in [0.5, 1)
  return 15 - e;
}

// Byte k of w placed in bits 8..15 of the lane's table base (bits 0..7 and
// 16..31 of `base`): the lookup address of code byte k.
template <int K>
__device__ __forceinline__ uint32_t lut_addr(uint32_t w, uint32_t base) {
  return __builtin_amdgcn_perm(w, base, 0x03020000u | ((4u + K) << 8));
}
__device__ __forceinline__ uint32_t lut_addr_dyn(uint32_t w, uint32_t base, int k) {
  switch (k & 3) {
    case 0:
      return lut_addr<0>(w, base);
    case 1:
      return lut_addr<1>(w, base);
    case 2:
      return lut_addr<2>(w, base);
    default:
      return lut_addr<3>(w, base);
  }
}

__device__ __forceinline__ uint2 lds_read_u2(const uint8_t* smem, uint32_t addr) {
  return *reinterpret_cast<const uint2*>(smem + addr);
}
__device__ __forceinline__ uint4 lds_read_u4(const uint8_t* smem, uint32_t addr) {
  return *reinterpret_cast<const uint4*>(smem + addr);
}

__device__ __forceinline__ f16x8 as_f16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(f16x8, u32x4{a, b, c, d});
}

// Table entry e of one stream from its two centroids ce0 = c[e & 15],
// ce1 = c[e >> 4], scaled by 2^sh: key table (hi(ce0), hi(ce1)),
// (lo(ce0), lo(ce1)) (two dims of one token), value table (hi(ce0),
// lo(ce0)), (hi(ce1), lo(ce1)) (one dim of two tokens).
// The split of one centroid scaled by 2^sh: hi = f16(c 2^sh) in the low half,
// lo = f16(c 2^sh - hi) in the high half.  Lane j of a writer computes the
// split of the centroid it holds; table entries are then byte permutations of
// two or four such words.
__device__ __forceinline__ uint32_t centroid_split(float c, int sh) {
  const float x = ldexpf(c, sh);
  const _Float16 hi = static_cast<_Float16>(x);
  const _Float16 lo = static_cast<_Float16>(x - static_cast<float>(hi));
  return pack_f16x2(hi, lo);
}
// (hi a, hi b) and (lo a, lo b) from the splits a, b: the key table's k-slot pairs.
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// Writes both tables from the centroids: writer wavefront w (0..W-1, W = 8
// or 4) fills the 1 KB spans w, w + W, ..., w + 128 - W; in span s lane l
// writes the 16 bytes at 1 KB * s + 16 l, two copies of entry
// e = 4 (s % 64) + l / 16 of table s / 64 (keys, then values).  The entry's
// centroids are c[e % 16] = c[4 (s % 4) + l / 16], fixed for the wavefront
// (s % 4 = w % 4, W being a multiple of 4), and c[e / 16] = c[(s / 4) % 16],
// uniform over the span.  cvec: lane j < 16 holds key centroid j, lane 16 + j
// value centroid j.  Each write covers 1 KB contiguously (no bank conflicts).
template <int W>
__device__ __forceinline__ void write_tables(uint8_t* smem, float cvec, int sh_k, int sh_v, int w, int lane) {
  constexpr int kSpans = 2 * kTableBytes / 1024;
  constexpr int kPer = kSpans / W;
  static_assert(W % 4 == 0 && kSpans % W == 0 && kPer % 2 == 0, "spans split evenly, keys then values");
  const int src0 = 4 * (w & 3) + (lane >> 4);
  const int pair = static_cast<int>(centroid_split(cvec, lane < 16 ? sh_k : sh_v));
  const uint32_t p0k = __shfl(pair, src0), p0v = __shfl(pair, 16 + src0);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int span = w + W * k;
    const bool key = k < kPer / 2;
    const uint32_t p1 = __builtin_amdgcn_readlane(pair, (key ? 0 : 16) + ((span >> 2) & 15));
    // key entry (hi c0, hi c1), (lo c0, lo c1); value entry (hi c0, lo c0), (hi c1, lo c1)
    const uint2 e = key ? make_uint2(hi_pair(p0k, p1), lo_pair(p0k, p1)) : make_uint2(p0v, p1);
    *reinterpret_cast<uint4*>(smem + (span << 10) + (lane << 4)) = make_uint4(e.x, e.y, e.x, e.y);
  }
}

// 2-bit tables: entry e (one code byte: four codes c_r = (e >> 2r) & 3) is
// 16 bytes, replicated 16 times (copy c at e * 256 + c * 16, so a lane's
// 16-byte read of copy lane % 16 is conflict-free whatever the codes).  Key
// entry: (hi c_0, hi c_1), (lo c_0, lo c_1), (hi c_2, hi c_3), (lo c_2, lo c_3)
// -- four dims of one token, the k-slot order of one score product.  Value
// entry: (hi c_r, lo c_r) for r = 0..3 -- one dim of four tokens.  Span and
// entry numbering as in write_tables (e = 4 (s % 64) + l / 16): c_0 =
// c[l / 16] is fixed per lane, c_1 = c[s % 4], c_2 = c[(s / 4) % 4], c_3 =
// c[(s / 16) % 4] are uniform over the span.  cvec: lane j < 16 holds key
// centroid j % 4, lane 16 + j value centroid j % 4.
template <int W>
__device__ __forceinline__ void write_tables2(uint8_t* smem, float cvec, int sh_k, int sh_v, int w, int lane) {
  constexpr int kSpans = 2 * kTableBytes / 1024;
  constexpr int kPer = kSpans / W;
  static_assert(kSpans % W == 0 && kPer % 2 == 0, "spans split evenly, keys then values");
  const int g = lane >> 4;
  const int pair = static_cast<int>(centroid_split(cvec, lane < 16 ? sh_k : sh_v));
  const uint32_t p0k = __shfl(pair, g), p0v = __shfl(pair, 16 + g);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int span = w + W * k;
    const bool key = k < kPer / 2;
    const int tb = key ? 0 : 16;
    const uint32_t p[4] = {key ? p0k : p0v, static_cast<uint32_t>(__builtin_amdgcn_readlane(pair, tb + (span & 3))),
                           static_cast<uint32_t>(__builtin_amdgcn_readlane(pair, tb + ((span >> 2) & 3))),
                           static_cast<uint32_t>(__builtin_amdgcn_readlane(pair, tb + ((span >> 4) & 3)))};
    const uint4 e = key ? make_uint4(hi_pair(p[0], p[1]), lo_pair(p[0], p[1]), hi_pair(p[2], p[3]), lo_pair(p[2], p[3]))
                        : make_uint4(p[0], p[1], p[2], p[3]);
    *reinterpret_cast<uint4*>(smem + (span << 10) + (lane << 4)) = e;
  }
}

}  // namespace mx

template <int D, bool QF16, int BITS = 4>
__global__ __launch_bounds__(mx::threads_of<D>()) __attribute__((
    amdgpu_waves_per_eu(mx::waves_of<D>() / 4, mx::waves_of<D>() / 4))) void decode_mx_kernel(
    const DecodeArgs a) {
  using namespace mx;
  static_assert(D == 64 || D == 128 || D == 256, "head_dim 64, 128 or 256");
  static_assert(BITS == 4 || (BITS == 2 && D == 128), "4-bit rows, or 2-bit rows at head_dim 128");
  constexpr bool B2 = BITS == 2;      // 2-bit rows: 16-byte table entries, one per code byte
  constexpr int ROW = D * BITS / 8;   // packed bytes per row
  constexpr int KB = ROW / 4;         // key bytes per lane per tile (a quarter row)
  constexpr int KW = (KB + 3) / 4;    // key dwords per lane (KB = 8, 16, 32)
  constexpr int NS = D / 16;          // score products per tile
  constexpr int NV = D / 16;          // value products per tile
  constexpr int VW = D == 256 ? 2 : 1;  // value dwords per lane per row
  constexpr int E = D / kWave;
  constexpr int NW = waves_of<D>();   // wavefronts
  // A row is processed in NH halves at head_dim 256 (key lookups and score
  // products of dims [0, 128) then [128, 256) of each lane's quarter row;
  // value lookups and products of dims [0, 128) then [128, 256)), so that
  // only half a tile's lookups are live at a time.
  constexpr int NH = D == 256 ? 2 : 1;
  constexpr int KBH = KB / NH;        // key bytes (lookups) per half
  constexpr int NSH = NS / NH;        // score products per half
  constexpr int NVH = NV / NH;        // value products per half
  using L = Smem<D>;

  __shared__ __align__(16) uint8_t smem[L::kTotal];
  uint16_t* s_qb = reinterpret_cast<uint16_t*>(smem + L::kQb);  // [8][D] f16 bits
  float* s_q = reinterpret_cast<float*>(smem + L::kQ);           // [4][D]
  float* s_cur = reinterpret_cast<float*>(smem + L::kCur);       // [2][D]
  uint8_t* s_codes = smem + L::kCur + 2 * D * 4;                 // [2][D]
  float* s_misc = reinterpret_cast<float*>(smem + L::kMiscOff);  // [0..3] score scale per head, [4] output scale

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: row ranges and resources stay scalar
  const int n = lane & 15, g = lane >> 4;

  // ---- work item: grid (split, head group, layer x KV head), so no
  // division is needed; the query heads of (lkv, hg) start at lkv * group +
  // 4 hg of the [L * Hq] rows.
  const int split = blockIdx.x, hg = blockIdx.y, lkv = blockIdx.z;
  const int64_t qhg0 = static_cast<int64_t>(lkv) * a.group + hg * 4;

  // Rows: blocks of kStride rows dealt out cyclically over the splits (split
  // s takes blocks s, s + n, s + 2n, ...), each block cut into
  // kTilesPerBlock tiles of 16 rows.  Tile k of this split is tile
  // k % kTilesPerBlock of its (k / kTilesPerBlock)-th block.  The tiles are
  // dealt statically: wavefront w takes tiles w, w + NW, w + 2 NW, ..., so
  // every call sums the same tiles in the same order and returns the same
  // bits (a claim counter in LDS that let a wavefront running ahead take
  // more tiles measured the same: M 12.02-12.19 against 11.80-12.12 us
  // mean, C4 20.55-20.60 against 20.68-20.82).  Row offsets are 32-bit (the
  // host keeps capacity * ROW < 2^31).
  const int t1 = static_cast<int>(a.seq_len);
  const int row_splits = a.new_k != nullptr ? a.row_splits : a.n_splits;  // splits that read rows
  const int BSTRIDE = row_splits * kStride;
  const int n_blocks = (t1 + kStride - 1) / kStride;
  // In append mode split 0 also packs the new token: as in decode_kernel it
  // reads no rows where splits 1.. (row_splits of them) can take every block
  // without a longer share, and takes the lightest share (the blocks split
  // n_splits - 1 would take) otherwise, splits 1.. then taking the shares
  // of splits 0.. (4-layer decode loop at 32768 + t tokens x 8 KV heads, 32
  // splits: 65.0-65.8 -> 62.2-62.4 us per step for the lightest share).
  const int deal = a.new_k == nullptr ? split : split > 0 ? split - 1 : row_splits < a.n_splits ? n_blocks : a.n_splits - 1;
  const int n_iter = deal < n_blocks ? (n_blocks - deal + row_splits - 1) / row_splits : 0;
  const int n_tiles = n_iter * kTilesPerBlock;
  auto tile_row = [&](int k) {
    const unsigned uk = static_cast<unsigned>(k);
    return deal * kStride + static_cast<int>(uk / kTilesPerBlock) * BSTRIDE + static_cast<int>(uk % kTilesPerBlock) * kTile;
  };
  const uint8_t* kbase = a.k + static_cast<int64_t>(lkv) * a.cap * ROW;
  const uint8_t* vbase = a.v + static_cast<int64_t>(lkv) * a.cap * ROW;

  // Per-lane load offsets inside a tile: key quarter g of row n; value dword
  // n (and 16 + n at D = 256; dword n / 2 at D = 64) of rows 4g + r.
  const int koff = n * ROW + g * KB;
  constexpr int RW = ROW / 4;  // dwords per row
  const int voff = (4 * g) * ROW + 4 * (RW >= 16 ? n : (n >> 1));
  struct Raw {
    uint32_t k[KW];
    uint32_t v[4][VW];
  };
  auto load_tile = [&](int k, Raw& r) {
    const int row0 = min(tile_row(k), t1);
    const uint32_t bytes = static_cast<uint32_t>(t1 - row0) * ROW;
    const BufferRsrc rk = make_rsrc(kbase + static_cast<int64_t>(row0) * ROW, bytes);
    const BufferRsrc rv = make_rsrc(vbase + static_cast<int64_t>(row0) * ROW, bytes);
    if constexpr (KW == 2) {
      const u32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(rk, koff, 0, kRowLoadPolicy);
      r.k[0] = x.x;
      r.k[1] = x.y;
    } else {
#pragma unroll
      for (int q = 0; q < KW / 4; ++q) {
        const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(rk, koff + 16 * q, 0, kRowLoadPolicy);
        r.k[4 * q] = x.x;
        r.k[4 * q + 1] = x.y;
        r.k[4 * q + 2] = x.z;
        r.k[4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int q = 0; q < VW; ++q) r.v[rr][q] = __builtin_amdgcn_raw_buffer_load_b32(rv, voff + rr * ROW + 64 * q, 0, kRowLoadPolicy);
  };

  // ---- set-up loads first (centroids, query, signs, appended token), then
  // the first tiles' rows: vector loads return in order, so a set-up value
  // requested after the rows would wait for them.
  // centroids in lanes: lane j < 16 key centroid j, lane 16 + j value centroid j
  constexpr int NC = 1 << BITS;  // centroids per table
  const float* cptr = lane < 16 ? a.cent_k + (lane & (NC - 1)) : a.cent_v + (lane & (NC - 1));
  const float cvec = lane < 32 ? *cptr : 0.f;
  const bool appending = a.new_k != nullptr;
  const bool appender = appending && split == 0 && wave < 2;
  constexpr int kLevels = NC - 1;
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
  float qe[E], sg_first[E], sg_second[E];
  if (wave < 4) {
    const int64_t qoff = (qhg0 + wave) * D + lane * E;
#pragma unroll
    for (int i = 0; i < E; ++i)
      qe[i] = QF16 ? __half2float(static_cast<const __half*>(a.q)[qoff + i]) : static_cast<const float*>(a.q)[qoff + i];
  }
  if ((wave < 4 && (a.rotate_query || a.inverse_output)) || appender) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      sg_first[i] = a.signs_right[lane * E + i];
      sg_second[i] = a.signs_left[lane * E + i];
    }
  }

  constexpr int NR = kPrefetch + 1;
  Raw ring[NR];
  int kq[NR];  // tile held by each ring slot (wavefront-uniform)
  auto prefetch = [&]() {
#pragma unroll
    for (int j = 0; j < kPrefetch; ++j) {
      kq[j] = j * NW + wave;
      load_tile(kq[j], ring[j]);
    }
  };
  // The query wavefronts issue their first tiles' rows right after their
  // set-up loads (which return first): the memory starts streaming while
  // the set-up runs.  The table writers issue theirs after writing, since a
  // wavefront whose loads cannot issue (every CU's rows in flight) stalls,
  // and the tables gate the set-up barrier.  Measured at M: split kernel
  // median 11.9 -> 11.4 us; C3 and C4 unchanged.
  if (wave < 4) prefetch();
  __builtin_amdgcn_sched_barrier(0);
  int next_tile = kPrefetch * NW + wave;  // the wavefront's next tile after its prefetched ones
  auto claim = [&]() {
    const int k = next_tile;
    next_tile += NW;
    return k;
  };

  // power-of-two scales of the two tables (lane rows 0 and 1 hold their centroids)
  const int sh_lane = scale_shift(group_reduce<16, OpMax>(fabsf(cvec)));
  const int sh_k = __builtin_amdgcn_readlane(sh_lane, 0), sh_v = __builtin_amdgcn_readlane(sh_lane, 16);
  if (wave >= 4) {
    if constexpr (B2)
      write_tables2<NW - 4>(smem, cvec, sh_k, sh_v, wave - 4, lane);
    else
      write_tables<NW - 4>(smem, cvec, sh_k, sh_v, wave - 4, lane);
  }
  if (wave == 4 && lane == 0) s_misc[4] = ldexpf(1.f, -(sh_v + 7));  // weights carry 2^7, values 2^sh_v

  // ---- append mode: rotate (as on append) and quantize the new token.
  if (appender) {
    if (wave == 1 ? a.rotate_new_v : a.rotate_new_k) wave_rotate_signs<D>(tok, sg_first, sg_second, a.sqrt_d);
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const uint32_t code = quantize_count<BITS>(tok[i], bnd);
      s_codes[wave * D + lane * E + i] = static_cast<uint8_t>(code);
      s_cur[wave * D + lane * E + i] = (wave == 0 ? a.cent_k : a.cent_v)[code];
    }
  }

  // ---- queries: optional rotation (bit-identical to the reference), the
  // softmax scale and log2(e) folded in (scores come out in log2 units), then
  // the exact f16 split of q * 2^shift.
  if (wave < 4) {
    if (a.rotate_query) wave_rotate_signs<D>(qe, sg_first, sg_second, a.sqrt_d);
    float mxq = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      qe[i] *= a.q_scale;
      s_q[wave * D + lane * E + i] = qe[i];
      mxq = fmaxf(mxq, fabsf(qe[i]));
    }
    mxq = group_reduce<kWave, OpMax>(mxq);
    const int sh_q = scale_shift(mxq);
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float x = ldexpf(qe[i], sh_q);
      const _Float16 h = static_cast<_Float16>(x);
      const _Float16 l = static_cast<_Float16>(x - static_cast<float>(h));
      s_qb[wave * L::kQbStride + lane * E + i] = __builtin_bit_cast(uint16_t, h);
      s_qb[(4 + wave) * L::kQbStride + lane * E + i] = __builtin_bit_cast(uint16_t, l);
    }
    if (lane == 0) s_misc[wave] = ldexpf(1.f, -(sh_q + sh_k));  // raw score -> log2 units
  }
  if (wave >= 4) prefetch();
  // the set-up exchanges data through LDS only: the barrier leaves the
  // prefetched rows in flight
  lds_barrier();
  if (appender) {
    constexpr int W = D * BITS / 32;
    if (hg == 0 && lane < W) {
      uint32_t* dst = (wave == 0 ? a.k_slab : a.v_slab) + (static_cast<int64_t>(lkv) * a.cap + a.seq_len) * W + lane;
      *dst = pack_word<BITS, D>(s_codes + wave * D, lane);
    }
  }

  // ---- this lane's query operands: column n (hi split of head n, lo split
  // of head n - 4, zero from 8), the g-th quarter of the dims; each pair of
  // dims fills the k-slots of both key parts (hi, lo).
  uint32_t qd[D / 8];  // f16 pairs of this lane's D / 4 dims
#pragma unroll
  for (int i = 0; i < D / 8; ++i)
    qd[i] = n < 8 ? reinterpret_cast<const uint32_t*>(s_qb + n * L::kQbStride + g * (D / 4))[i] : 0u;
  const float score_scale = s_misc[n & 3];
  const float out_scale = s_misc[4];

  // table bases (offsets into smem): copy lane % 32 of 8-byte entries
  // (4-bit) or lane % 16 of 16-byte entries (2-bit), key table at 0, value
  // table at 65536; bits 8..15 stay clear for the code byte
  const uint32_t base_k = B2 ? (lane & 15) * 16 : (lane & 31) * 8;
  const uint32_t base_v = base_k + kTableBytes;

  // Softmax state, log2 units.  Lane m works on head m % 4: m_lane is that
  // head's running maximum (wavefront-wide: every lane sharing m % 4 holds
  // the same value); bias = 7 - m_lane (the weights come out as p * 2^7, the
  // scale of their exact f16 split); l_lane is the lane's softmax sum in
  // units of 2^-7.
  float m_lane = -INFINITY;
  float bias = INFINITY;  // +inf forces a maximum on the first tile
  float l_lane = 0.f;
  const int kk = (lane >> 2) & 3;  // this lane's token within its lane group's 4
  f32x4v acc[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) acc[j] = f32x4v{0.f, 0.f, 0.f, 0.f};
  constexpr float kWeightExp = 7.f;  // weights carry 2^7

  // Per tile, in order: key lookups (KB table reads) and score products,
  // value lookups (NV x 2 table reads), softmax, value products.  The value
  // reads land while the softmax runs; the three wavefronts of a SIMD cover
  // each other's table-read and product latencies.  (Issuing all key reads
  // of a tile before its first score product speeds the oldest wavefronts
  // up but not the last one, and back-to-back split launches at M slow from
  // 13.4 to 14.1 us.)
  using KeyL = std::conditional_t<B2, uint4, uint2>;
  KeyL kl[KBH];       // key lookups of one half, one per byte of the lane's quarter row
  uint2 vl[NVH][2];   // 4-bit value lookups of one half: product j, token pair (0, 1) / (2, 3)
  uint4 vl4[B2 ? NVH : 1];  // 2-bit value lookups: product j, tokens 0..3
  auto key_lookups = [&](const Raw& r, int h) {
#pragma unroll
    for (int b = 0; b < KBH; ++b) {
      const uint32_t addr = lut_addr_dyn(r.k[(h * KBH + b) / 4], base_k, b & 3);
      if constexpr (B2)
        kl[b] = lds_read_u4(smem, addr);
      else
        kl[b] = lds_read_u2(smem, addr);
    }
  };
  // 2-bit values: lane (n, g) takes dims 8n .. 8n + 7 -- fields 8 (n & 1) + j
  // of dword n / 2 of rows 4g .. 4g + 3.  The fields of one dim in the four
  // rows are gathered into one byte (row r at bits 2r), the lookup key of the
  // value table; the four words below hold those bytes for all 16 fields of
  // the dword (field f in word f % 4, byte f / 4), and the lane's selectors
  // pick byte 2 (n & 1) (j < 4) or 2 (n & 1) + 1 (j >= 4).
  const uint32_t vsel0 = 0x03020000u | ((4u + 2u * (n & 1)) << 8);
  const uint32_t vsel1 = vsel0 + 0x100u;
  auto value_lookups2 = [&](const Raw& r) {
    const uint32_t h0 = r.v[0][0], h1 = r.v[1][0], h2 = r.v[2][0], h3 = r.v[3][0];
    // nibble k of P (Q): field 2k (2k + 1) of rows 0 and 1; P2, Q2 rows 2 and 3
    const uint32_t P = (h0 & 0x33333333u) | ((h1 << 2) & 0xccccccccu);
    const uint32_t Q = ((h0 >> 2) & 0x33333333u) | (h1 & 0xccccccccu);
    const uint32_t P2 = (h2 & 0x33333333u) | ((h3 << 2) & 0xccccccccu);
    const uint32_t Q2 = ((h2 >> 2) & 0x33333333u) | (h3 & 0xccccccccu);
    const uint32_t F[4] = {(P & 0x0f0f0f0fu) | ((P2 << 4) & 0xf0f0f0f0u),     // fields 0, 4, 8, 12
                           (Q & 0x0f0f0f0fu) | ((Q2 << 4) & 0xf0f0f0f0u),     // fields 1, 5, 9, 13
                           ((P >> 4) & 0x0f0f0f0fu) | (P2 & 0xf0f0f0f0u),     // fields 2, 6, 10, 14
                           ((Q >> 4) & 0x0f0f0f0fu) | (Q2 & 0xf0f0f0f0u)};    // fields 3, 7, 11, 15
#pragma unroll
    for (int j = 0; j < NVH; ++j)
      vl4[j] = lds_read_u4(smem, __builtin_amdgcn_perm(F[j & 3], base_v, j < 4 ? vsel0 : vsel1));
  };
  // value dword q = h of the lane's rows (dims 128 h + 8 n .. + 7; D = 64:
  // the n & 1 half of dword n / 2)
  auto value_lookups = [&](const Raw& r, int h) {
    if constexpr (B2) {
      value_lookups2(r);
    } else {
      const int q = h;
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        uint32_t w0 = r.v[2 * pr][q], w1 = r.v[2 * pr + 1][q];
        if constexpr (D == 64) {
          w0 = (n & 1) ? (w0 >> 16) : (w0 & 0xffffu);
          w1 = (n & 1) ? (w1 >> 16) : (w1 & 0xffffu);
        }
        // nibbles of one dim in two tokens interleaved into one byte
        const uint32_t ev = (w0 & 0x0f0f0f0fu) | ((w1 << 4) & 0xf0f0f0f0u);
        const uint32_t od = ((w0 >> 4) & 0x0f0f0f0fu) | (w1 & 0xf0f0f0f0u);
        constexpr int JN = D == 64 ? 4 : 8;  // dims per dword this lane uses
        static_assert(JN == NVH, "one value product per dim of the dword");
#pragma unroll
        for (int jj = 0; jj < JN; ++jj)
          vl[jj][pr] = lds_read_u2(smem, lut_addr_dyn((jj & 1) ? od : ev, base_v, jj >> 1));
      }
    }
  };
  auto scores = [&](f32x4v& ds, int h) {
#pragma unroll
    for (int s2 = 0; s2 < NSH; ++s2) {
      const int q2 = 2 * (h * NSH + s2);
      f16x8 A;
      if constexpr (B2)
        A = __builtin_bit_cast(f16x8, kl[s2]);
      else
        A = as_f16x8(kl[2 * s2].x, kl[2 * s2].y, kl[2 * s2 + 1].x, kl[2 * s2 + 1].y);
      const f16x8 B = as_f16x8(qd[q2], qd[q2], qd[q2 + 1], qd[q2 + 1]);
      ds = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, ds, 0, 0, 0);
    }
  };
  // Softmax and value products of tile k.  After the score products lane
  // (n, g) holds column n of tokens 4g + rr; column h + column h + 4 is head
  // h's score (hi + lo query split, a row_ror:12 add), valid on lanes n < 4.
  // The four registers are then spread over the row, so that lane m holds
  // one score: head m % 4, token 4g + m / 4 % 4; the softmax runs once per
  // lane, and the weights are gathered back into the A operand of the value
  // products: row h (lanes n = h) the hi splits of head h's 4 tokens, row
  // 4 + h their lo splits, each as an f16 pair (w, w) facing the value's
  // (hi, lo) k-slots.  Rows 8..15 carry junk weights whose output rows are
  // never read.  Only a split's last tiles can be partial.
  auto softmax = [&](const f32x4v& ds, int k) {
    float s4[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) s4[rr] = ds[rr] + dpp_move<kDppRor12>(ds[rr]);
    float sc = s4[0];  // bank b (lanes 4b .. 4b + 3) takes register b from lanes 0..3
    sc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, sc), __builtin_bit_cast(int, s4[1]),
                                                               0x114, 0xf, 0x2, false));  // row_shr:4
    sc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, sc), __builtin_bit_cast(int, s4[2]),
                                                               0x118, 0xf, 0x4, false));  // row_shr:8
    sc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, sc), __builtin_bit_cast(int, s4[3]),
                                                               0x11C, 0xf, 0x8, false));  // row_shr:12
    const int row0 = tile_row(k);
    const bool full = row0 + kTile <= t1;  // wavefront-uniform
    const bool valid = full || row0 + 4 * g + kk < t1;
    float z = fmaf(sc, score_scale, bias);
    if (!full) z = valid ? z : -INFINITY;
    if (__builtin_amdgcn_ballot_w64(z > kRescaleThreshold + kWeightExp) != 0) {
      // a running maximum moves: wavefront-wide per head (lanes sharing
      // lane % 4); accumulators of head rr (rows rr, 4 + rr) rescaled
      float mx = valid ? sc * score_scale : -INFINITY;
      mx = strided_reduce<4, OpMax>(mx);
      float alpha = 1.f;
      if (mx > m_lane + kRescaleThreshold) {
        alpha = fast_exp2(m_lane - mx);  // 0 before the first maximum
        m_lane = mx;
      }
      l_lane *= alpha;
      bias = kWeightExp - m_lane;
      const f32x4v al = {quad_broadcast_t<0>(alpha), quad_broadcast_t<1>(alpha), quad_broadcast_t<2>(alpha),
                         quad_broadcast_t<3>(alpha)};
#pragma unroll
      for (int j = 0; j < NV; ++j) acc[j] *= al;
      z = valid ? fmaf(sc, score_scale, bias) : -INFINITY;
    }
    const float p = fast_exp2(z);  // p * 2^7
    l_lane += p;
    // exact split of p * 2^7: hi = low 13 mantissa bits cleared, lo = rest
    const float ph = __uint_as_float(__float_as_uint(p) & 0xffffe000u);
    const int whi = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pkrtz(ph, ph));
    const int wlo = __builtin_bit_cast(int, __builtin_amdgcn_cvt_pkrtz(p - ph, p - ph));
    // gather: A register r holds token r of the lane group; lanes 0..3 read
    // the hi pair of lane n + 4r, lanes 4..7 the lo pair of lane n - 4 + 4r
    const int a0 = __builtin_amdgcn_update_dpp(whi, wlo, 0x114, 0xf, 0x2, false);  // row_shr:4 into lanes 4..7
    int a1 = __builtin_amdgcn_update_dpp(wlo, whi, 0x104, 0xf, 0x1, false);         // row_shl:4 into lanes 0..3
    int a2 = __builtin_amdgcn_update_dpp(whi, whi, 0x108, 0xf, 0x1, false);         // row_shl:8 into lanes 0..3
    a2 = __builtin_amdgcn_update_dpp(a2, wlo, 0x104, 0xf, 0x2, false);              // row_shl:4 into lanes 4..7
    int a3 = __builtin_amdgcn_update_dpp(whi, whi, 0x10C, 0xf, 0x1, false);         // row_shl:12 into lanes 0..3
    a3 = __builtin_amdgcn_update_dpp(a3, wlo, 0x108, 0xf, 0x2, false);              // row_shl:8 into lanes 4..7
    return as_f16x8(static_cast<uint32_t>(a0), static_cast<uint32_t>(a1), static_cast<uint32_t>(a2),
                    static_cast<uint32_t>(a3));
  };
  auto value_products = [&](const f16x8& Aw, int h) {
#pragma unroll
    for (int j = 0; j < NVH; ++j) {
      f16x8 B;
      if constexpr (B2)
        B = __builtin_bit_cast(f16x8, vl4[j]);
      else
        B = as_f16x8(vl[j][0].x, vl[j][0].y, vl[j][1].x, vl[j][1].y);
      acc[h * NVH + j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Aw, B, acc[h * NVH + j], 0, 0, 0);
    }
  };

  // Tiles past the split's end load nothing and read as masked tiles; a
  // wavefront's tiles only grow, so it stops at its first such tile.  The
  // stages of a tile run in order; the three wavefronts of a SIMD overlap
  // each other's table-read and product latencies.
  bool more = kq[0] < n_tiles;
  int claimed = claim();
  while (more) {
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int nx = (j + kPrefetch) % NR;
      kq[nx] = claimed;
      load_tile(kq[nx], ring[nx]);
      claimed = claim();
      f32x4v ds = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        key_lookups(ring[j], h);
        scores(ds, h);
      }
      value_lookups(ring[j], 0);
      const f16x8 Aw = softmax(ds, kq[j]);
      value_products(Aw, 0);
#pragma unroll
      for (int h = 1; h < NH; ++h) {
        value_lookups(ring[j], h);
        value_products(Aw, h);
      }
      if (kq[(j + 1) % NR] >= n_tiles) {
        more = false;
        break;
      }
    }
  }

  // ---- combine: rows h and 4 + h (lane groups 0 and 1), then the
  // wavefronts.  Lane n of group 0 holds head rr's output at dims of column n.
  if constexpr (!L::kRedApart) __syncthreads();  // the tables are dead: reuse their space
  // s_red: [NW x 4 heads] rows of RS floats; dim d of a row sits at
  // d + 4 (d / 64), and RS = 2 (mod 4) and above that, so that the 32 lanes writing one
  // register pair (16 dims x 2 rows) hit 32 distinct banks
  constexpr int RS = L::kRS;
  float* s_red = reinterpret_cast<float*>(smem + L::kRed);
  float* s_mw = reinterpret_cast<float*>(smem + L::kRed + NW * 4 * RS * 4);  // [NW][4]
  float* s_lw = s_mw + NW * 4;                                       // [NW][4]
  auto red_pos = [](int d) { return d + 4 * (d >> 6); };
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    // dim of column n in product j: 128 (j / 8) + 8n + j % 8 (D = 128, 256), 4n + j (D = 64)
    const int dim = D == 64 ? 4 * n + j : 128 * (j / 8) + 8 * n + (j % 8);
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      // rows h (hi weights) and 4 + h (lo weights) of head h are lane groups
      // 0 and 1; one permlane16 swap sums two registers: group 0 receives
      // head 2pr's sum, group 1 head 2pr + 1's
      const LanePair r = permlane_swap<16>(acc[j][2 * pr], acc[j][2 * pr + 1]);
      if (g < 2) s_red[(wave * 4 + 2 * pr + g) * RS + red_pos(dim)] = r.first + r.second;
    }
  }
  {
    const float lw = strided_reduce<4, OpSum>(l_lane) * (1.f / 128.f);  // head lane % 4
    if (lane < 4) {
      s_mw[wave * 4 + lane] = m_lane;
      s_lw[wave * 4 + lane] = lw;
    }
  }
  lds_barrier();  // the wavefronts' partials meet in LDS

  auto wave_weights = [&](int h, float (&f)[NW]) {
    float M = s_mw[h];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, s_mw[w * 4 + h]);
#pragma unroll
    for (int w = 0; w < NW; ++w) f[w] = s_mw[w * 4 + h] == -INFINITY ? 0.f : fast_exp2(s_mw[w * 4 + h] - M);
    return M;
  };
  if (wave < 4) {
    float f[NW];
    const float M = wave_weights(wave, f);
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) l = fmaf(s_lw[w * 4 + wave], f[w], l);
    float e[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v = fmaf(s_red[(w * 4 + wave) * RS + red_pos(lane * E + i)], f[w], v);
      e[i] = v * out_scale;
    }
    if (a.n_splits == 1) {
      // one split: finish the row here (current token, normalisation, inverse rotation)
      float* row = s_red + wave * RS;  // row (wave 0, head `wave`): read only by this wavefront
#pragma unroll
      for (int i = 0; i < E; ++i) row[lane * E + i] = e[i];
      const float* ck = appending ? s_cur : a.cur_k ? a.cur_k + static_cast<int64_t>(lkv) * D : nullptr;
      const float* cv = appending ? s_cur + D : a.cur_v ? a.cur_v + static_cast<int64_t>(lkv) * D : nullptr;
      finish_row<D>(row, M, l, s_q + wave * D, ck, cv, a.inverse_output, sg_second, sg_first, a.sqrt_d,
                    a.out + (qhg0 + wave) * D);
    } else {
      // several splits: publish this split's (max, sum, accumulator rotated back)
      if (a.inverse_output) wave_rotate_signs<D>(e, sg_second, sg_first, a.sqrt_d);
      float* dst = a.ws_acc + ((qhg0 + wave) * a.n_splits + split) * D + lane * E;
#pragma unroll
      for (int i = 0; i < E; ++i) dst[i] = e[i];
      if (lane == 0) {
        a.ws_ml[((qhg0 + wave) * a.n_splits + split) * 2] = M;
        a.ws_ml[((qhg0 + wave) * a.n_splits + split) * 2 + 1] = l;
      }
      if (split == 0 && (appending || a.cur_k != nullptr)) {
        const float* ck = (appending ? s_cur : a.cur_k + static_cast<int64_t>(lkv) * D) + lane * E;
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < E; ++i) dot = fmaf(s_q[wave * D + lane * E + i], ck[i], dot);
        dot = group_sum<kWave>(dot);
        if (lane == 0) a.ws_cur_s[qhg0 + wave] = dot;
        if (wave == 0 && hg == 0) {
          float v[E];
          const float* cv = (appending ? s_cur + D : a.cur_v + static_cast<int64_t>(lkv) * D) + lane * E;
#pragma unroll
          for (int i = 0; i < E; ++i) v[i] = cv[i];
          if (a.inverse_output) wave_rotate_signs<D>(v, sg_second, sg_first, a.sqrt_d);
#pragma unroll
          for (int i = 0; i < E; ++i) a.ws_cur_v[static_cast<int64_t>(lkv) * D + lane * E + i] = v[i];
        }
      }
    }
  }
}
