// Device-side helpers shared by the quantized paged-KV kernels (gfx950, wave64).
//
// Numerics that must be bit-identical to the CPU restatement of the reference
// (K rotation, RTN int8, Lloyd-Max V codec) are implemented here with a fixed
// operation order; see the comments on each helper.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace s8kv {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

#define S8KV_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Buffer resources: every bulk cache access goes through a buffer descriptor
// whose num_records is the tensor's byte size, so an index that escapes the
// tensor reads zeros instead of faulting.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// Pools past 4 GiB: a descriptor over a tensor's bytes from the wave-uniform
// 64-bit offset `off` on (at most 4 GiB - 1 of them, none past the end), so a
// tile's or a row's accesses keep 32-bit offsets from a base rebased per tile.
__device__ __forceinline__ rsrc_t window_rsrc(const void* base, uint64_t total, uint64_t off) {
  const uint64_t rem = off < total ? total - off : 0;
  return make_rsrc(static_cast<const char*>(base) + off, (uint32_t)(rem < 0xFFFFFFFFull ? rem : 0xFFFFFFFFull));
}
// `off` is the per-lane (VGPR) byte offset, `soff` a wave-uniform (SGPR) one.
// AUX is the cache-policy operand: 0, or kNT for data streamed once (the
// loads are marked non-temporal, so they do not displace reused lines in the
// caches; a read-only sweep over the decode's tiles reads ~12 % faster so).
constexpr int kNT = 2;
template <int AUX = 0>
__device__ __forceinline__ u32x4_t bload128(rsrc_t r, uint32_t off, uint32_t soff = 0) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, AUX));
}
template <int AUX = 0>
__device__ __forceinline__ u32x2_t bload64(rsrc_t r, uint32_t off, uint32_t soff = 0) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, soff, AUX));
}
// Three consecutive dwords (a K8V3 code group's bit-plane words) in one load.
template <int AUX = 0>
__device__ __forceinline__ u32x3_t bload96(rsrc_t r, uint32_t off, uint32_t soff = 0) {
  return __builtin_bit_cast(u32x3_t, __builtin_amdgcn_raw_buffer_load_b96(r, off, soff, AUX));
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t bload32(rsrc_t r, uint32_t off, uint32_t soff = 0) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, soff, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ float4_t bloadf4(rsrc_t r, uint32_t off, uint32_t soff = 0) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, AUX));
}
template <int AUX = 0>
__device__ __forceinline__ void bstore128(u32x4_t v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v), r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ void bstore32(uint32_t v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ void bstore8(uint8_t v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b8(v, r, off, 0, AUX);
}

// ---------------------------------------------------------------------------
// Cross-lane helpers (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  int lane = __lane_id();
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, v)));
}

// Exchanges across lane ^ 16 and lane ^ 32 on the VALU (gfx950
// v_permlane16_swap / v_permlane32_swap, both operands x): the two results
// hold {x, x of lane ^ m} -- own value first in lanes with bit m clear,
// partner first in lanes with bit m set.
struct LanePair { float a, b; };
__device__ __forceinline__ LanePair lane_pair16(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ LanePair lane_pair32(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
// max / sum with the value of lane ^ 16 (or ^ 32); fmax and + are
// commutative, so the result equals the shuffle-based form bit for bit.
__device__ __forceinline__ float max_x16(float x) { const LanePair p = lane_pair16(x); return fmaxf(p.a, p.b); }
__device__ __forceinline__ float max_x32(float x) { const LanePair p = lane_pair32(x); return fmaxf(p.a, p.b); }
__device__ __forceinline__ float sum_x16(float x) { const LanePair p = lane_pair16(x); return p.a + p.b; }
__device__ __forceinline__ float sum_x32(float x) { const LanePair p = lane_pair32(x); return p.a + p.b; }
// Walsh-Hadamard butterfly across lane ^ 16 (^ 32): lanes with the bit clear
// get x + partner, lanes with it set get partner - x.  One FMA with a per-lane
// sign: fma(+1, b, a) = RN(a + b) and fma(-1, b, a) = RN(a - b), signed zeros
// included, so the result equals the add / subtract pair bit for bit.
__device__ __forceinline__ float butterfly_x16(float x, int lane) {
  const LanePair p = lane_pair16(x);
  return __builtin_fmaf((lane & 16) ? -1.0f : 1.0f, p.b, p.a);
}
__device__ __forceinline__ float butterfly_x32(float x, int lane) {
  const LanePair p = lane_pair32(x);
  return __builtin_fmaf((lane & 32) ? -1.0f : 1.0f, p.b, p.a);
}

// Walsh-Hadamard butterfly across lane ^ M on the VALU or the LDS swizzle
// unit (no lane-address registers): M = 1, 2 DPP quad permutes, M = 4 an LDS
// swizzle, M = 8 a DPP row rotate by 8, M = 16, 32 the permlane swaps.
// Lanes with bit M clear get x + partner, lanes with it set partner - x.
template <int M>
__device__ __forceinline__ float xor_partner(float x) {  // the value of lane ^ M, M = 1, 2, 4, 8
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "lane xor 1..8");
  const int u = __builtin_bit_cast(int, x);
  int pu;
  if constexpr (M == 1) pu = __builtin_amdgcn_mov_dpp(u, 0xB1, 0xF, 0xF, false);        // quad_perm [1,0,3,2]
  else if constexpr (M == 2) pu = __builtin_amdgcn_mov_dpp(u, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  else if constexpr (M == 4) pu = __builtin_amdgcn_ds_swizzle(u, 0x1F | (4 << 10));     // bit mode, xor 4
  else pu = __builtin_amdgcn_mov_dpp(u, 0x128, 0xF, 0xF, false);                        // row_ror:8
  return __builtin_bit_cast(float, pu);
}
template <int M>
__device__ __forceinline__ float butterfly_xor(float x, int lane) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane xor 1..32");
  if constexpr (M == 16) {
    return butterfly_x16(x, lane);
  } else if constexpr (M == 32) {
    return butterfly_x32(x, lane);
  } else {
    const float p = xor_partner<M>(x);
    return __builtin_fmaf((lane & M) ? -1.0f : 1.0f, x, p);  // x + p, or p - x
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f(v, m));
  return v;
}

// ---------------------------------------------------------------------------
// int8 -> fp16 conversion for MFMA operands (exact: |x| <= 128 fits fp16).
// Bytes are biased to unsigned (x ^ 0x80 = x + 128), placed in the mantissa of
// the fp16 constant 1024 (0x6400) with v_perm_b32, then 1152 is subtracted
// with one packed fp16 add per pair.
// ---------------------------------------------------------------------------
__device__ __forceinline__ half8_t i8x8_to_f16(u32x2_t x) {
  const uint32_t magic = 0x64646464u;
  uint32_t a = x.x ^ 0x80808080u;
  uint32_t b = x.y ^ 0x80808080u;
  u32x4_t w;
  w.x = __builtin_amdgcn_perm(magic, a, 0x04010400u);
  w.y = __builtin_amdgcn_perm(magic, a, 0x04030402u);
  w.z = __builtin_amdgcn_perm(magic, b, 0x04010400u);
  w.w = __builtin_amdgcn_perm(magic, b, 0x04030402u);
  half8_t h = __builtin_bit_cast(half8_t, w);
  const half8_t bias = {-1152.0f16, -1152.0f16, -1152.0f16, -1152.0f16,
                        -1152.0f16, -1152.0f16, -1152.0f16, -1152.0f16};
  return h + bias;
}

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Quantization helpers (must match the CPU restatement bit for bit)
// ---------------------------------------------------------------------------

// Materialize an fp32 value: stops the compiler from fusing the operation that
// produced it into a following fp16 conversion (v_fma_mix*), which would round
// once from the exact product instead of rounding to fp32 first.
__device__ __forceinline__ float materialize(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// An opaque copy of a per-lane value: values derived from it are recomputed
// where they are used instead of being hoisted out of enclosing loops (and
// held in VGPRs across them).
__device__ __forceinline__ int opaque_int(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// ---------------------------------------------------------------------------
// Exponent shift of the fp16 softmax weights
// ---------------------------------------------------------------------------
// The PV MFMAs take the weights p * (V scale | block norm) as fp16 hi + lo,
// whose range (2^-24 .. 65504) is far narrower than fp32's.  With p relative
// to the running max and scales near 2^-6, weights below ~2^-18 of the
// largest would underflow to zero -- and tens of thousands of such keys hold a
// visible share of the softmax mass.  A wave-uniform power-of-two shift
// `esh`, folded into the running max (the kernels keep m_ref = max - esh),
// scales every p by 2^esh such that the largest weight the lazy max allows,
// 2^(kMaxSlack + esh), times `vbound` (a power of two above every scale seen)
// is 2^15.  l and the accumulators carry the same factor, which cancels in
// acc / l and in the combine of partials (each is relative to its own m_ref).
//
// WeightShift holds esh and vbound (and the lazy-max threshold esh + slack)
// as integers and float bit patterns read back with readfirstlane, so that
// the loop-carried state stays in scalar registers.  raise(vmax): the tile's
// largest scale `vmax` (> vbound, finite, equal in every lane) raises the
// bound; returns the change of esh, by which l and acc are multiplied
// (2^change) and m_ref lowered.  esh stays within [-16, 64], which keeps
// l <= 2^28 keys * 2^(8 + 64) inside fp32.
struct WeightShift {
  int esh;
  uint32_t vbound_bits;  // 0: no scale seen yet
  uint32_t thr_bits;     // float(esh) + slack
  __device__ __forceinline__ explicit WeightShift(float slack)
      : esh(0), vbound_bits(0), thr_bits(__builtin_bit_cast(uint32_t, slack)) {}
  __device__ __forceinline__ float vbound() const { return __builtin_bit_cast(float, vbound_bits); }
  __device__ __forceinline__ float thr() const { return __builtin_bit_cast(float, thr_bits); }
  __device__ __forceinline__ int raise(float vmax, float slack) {
    const uint32_t vb = (uint32_t)__builtin_amdgcn_readfirstlane((int)__builtin_bit_cast(uint32_t, vmax));
    const int k = min((int)((vb >> 23) & 0xFFu) - 126, 128);  // vbound = 2^k > vmax (k = 128: +inf)
    const int sh = max(-16, min(64, 15 - (int)slack - k));
    const int d = sh - esh;
    esh = sh;
    vbound_bits = (uint32_t)(k + 127) << 23;
    thr_bits = (uint32_t)__builtin_amdgcn_readfirstlane((int)__builtin_bit_cast(uint32_t, (float)sh + slack));
    return d;
  }
};

// Round-half-even to int, clamped to [-127, 127].  `y` and `scale` are fp32;
// the division is IEEE correctly rounded (HIP's default fp32 divide).
__device__ __forceinline__ int rtn_i8(float y, float scale) {
  if (!(scale > 0.0f)) return 0;
  float q = __builtin_rintf(y / scale);
  q = fminf(127.0f, fmaxf(-127.0f, q));
  return (int)q;
}

// 1.5 * 2^23: adding it to a |t| < 2^22 rounds t half-even to an integer n
// (the fp32 spacing there is 1) and leaves n in the low bits of the sum's
// encoding, kRoundMagicBits + n; its low byte is n as an int8.
constexpr float kRoundMagic = 12582912.0f;
constexpr uint32_t kRoundMagicBits = 0x4B400000u;

// The reciprocal rtn_i8_recip takes: 1 / scale (IEEE), or 0 for a zero scale
// (an all-zero row), which makes every quotient of that row 0 without a
// per-element test.
__device__ __forceinline__ float rtn_rscale(float scale) { return scale > 0.0f ? 1.0f / scale : 0.0f; }

// rtn_i8 with the quotient from a per-row reciprocal: rscale = rtn_rscale(scale),
// q0 = RN(y * rscale), the residual y - q0 * scale exactly by FMA, and one FMA
// correction q0 + residual * rscale (Markstein's division).  For the append's
// operands -- y an fp16 value and scale = RN(m / 127) for an fp16 absmax
// m >= |y| -- the corrected quotient equals the IEEE quotient y / scale for
// every such pair and rounds to an integer in [-127, 127] (an exhaustive check
// over all 1.0e9 of them), so the codes equal rtn_i8's without its clamp.
// Returns kRoundMagicBits + code (rtn_i8_biased; low byte = the int8) or the
// code.  A NaN quotient (a row holding inf or NaN) gives code 0.
__device__ __forceinline__ uint32_t rtn_i8_biased(float y, float scale, float rscale) {
  const float q0 = materialize(y * rscale);
  const float r = __builtin_fmaf(-q0, scale, y);
  return __builtin_bit_cast(uint32_t, __builtin_fmaf(r, rscale, q0) + kRoundMagic);
}
__device__ __forceinline__ int rtn_i8_recip(float y, float scale, float rscale) {
  return (int)(rtn_i8_biased(y, scale, rscale) - kRoundMagicBits);
}

// Low bytes of four words, in order, as one word (three byte permutes).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0C0C0400u);
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x0C0C0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// ---------------------------------------------------------------------------
// One (token, head) row spread over a wave: lane l holds elements l, l+64, ...
// (rows shorter than 64 use the first D lanes).
// ---------------------------------------------------------------------------
template <int D>
struct RowLayout {
  static constexpr int E = D >= 64 ? D / 64 : 1;    // elements per lane
  static constexpr int ACTIVE = D >= 64 ? 64 : D;   // lanes holding data
};

// Fixed-order fp32 Walsh-Hadamard transform of one D-row spread over the wave:
// stages h = 1, 2, ..., D/2; the pair (i, i+h) with bit h of i clear becomes
// (x[i] + x[i+h], x[i] - x[i+h]).
template <int D, int H>
__device__ __forceinline__ void fwht_lane_stage(float (&x)[RowLayout<D>::E], int lane) {
  if constexpr (H < D && H < 64) {
#pragma unroll
    for (int j = 0; j < RowLayout<D>::E; ++j) x[j] = butterfly_xor<H>(x[j], lane);
  }
}
template <int D>
__device__ __forceinline__ void fwht_row(float (&x)[RowLayout<D>::E], int lane) {
  constexpr int E = RowLayout<D>::E;
  fwht_lane_stage<D, 1>(x, lane);  // h = 1 .. 32: across lanes
  fwht_lane_stage<D, 2>(x, lane);
  fwht_lane_stage<D, 4>(x, lane);
  fwht_lane_stage<D, 8>(x, lane);
  fwht_lane_stage<D, 16>(x, lane);
  fwht_lane_stage<D, 32>(x, lane);
#pragma unroll
  for (int hs = 1; hs < E; hs <<= 1) {  // h = 64*hs, in-lane
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if ((j & hs) == 0) {
        float a = x[j], b = x[j + hs];
        x[j] = a + b;
        x[j + hs] = a - b;
      }
    }
  }
}

template <int D>
__device__ __forceinline__ void load_row_f16(const _Float16* p, float (&x)[RowLayout<D>::E], int lane) {
  constexpr int E = RowLayout<D>::E;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    int e = lane + 64 * j;
    x[j] = (lane < RowLayout<D>::ACTIVE) ? (float)p[e] : 0.0f;
  }
}

// Per-row RTN int8 of the wave's row (lane layout of RowLayout): scale =
// absmax/127 over the wave, codes rint(y/scale) clamped to +-127 (y must be
// fp16 values: the quotient comes from rtn_i8_recip).
template <int D>
__device__ __forceinline__ float rtn_row(const float (&y)[RowLayout<D>::E], int (&q)[RowLayout<D>::E]) {
  constexpr int E = RowLayout<D>::E;
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < E; ++j) amax = fmaxf(amax, fabsf(y[j]));
  amax = wave_max(amax);
  const float scale = amax / 127.0f;
  const float rscale = rtn_rscale(scale);
#pragma unroll
  for (int j = 0; j < E; ++j) q[j] = rtn_i8_recip(y[j], scale, rscale);
  return scale;
}

// Codebooks for which lloyd3_search returns the first index minimising
// fl|u - c_j| for every |u| <= 1 (u = v / norm with norm >= |v|), or a NaN u
// (index 0, as the sequential scan): finite, c_0 >= -4, c_7 <= 4, ascending
// with neighbours at least 2^-19 apart.  Then for c_{j-1} < c_j <= u the
// exact distances differ by more than 2^-20 while each rounds by at most
// 2^-22, so the fp32 distances fall strictly up to the last c_j <= u and do
// not fall after the first minimum: "entry j is strictly nearer than entry
// j - 1" holds exactly for j = 1 .. m (m the first minimising index) and
// fails above m, so m is found by a binary search over j.
__device__ __forceinline__ bool lloyd3_search_ok(const float (&cb)[8]) {
  bool ok = cb[0] >= -4.0f && cb[7] <= 4.0f;
#pragma unroll
  for (int j = 1; j < 8; ++j) ok = ok && (cb[j] - cb[j - 1] >= 0x1p-19f);
  return ok;
}

// The bits of m for an 8-entry codebook accepted by lloyd3_search_ok: three
// tests of "entry j strictly nearer than entry j - 1" at j = 4, 4 b2 + 2 and
// 4 b2 + 2 b1 + 1, with the same fp32 distances as the sequential scan.
__device__ __forceinline__ void lloyd3_search(float u, const float (&cb)[8], bool& b2, bool& b1, bool& b0) {
  b2 = fabsf(u - cb[4]) < fabsf(u - cb[3]);
  const float c62 = b2 ? cb[6] : cb[2], c51 = b2 ? cb[5] : cb[1];
  const float c73 = b2 ? cb[7] : cb[3], c40 = b2 ? cb[4] : cb[0];
  b1 = fabsf(u - c62) < fabsf(u - c51);
  const float hi = b1 ? c73 : c51, lo = b1 ? c62 : c40;
  b0 = fabsf(u - hi) < fabsf(u - lo);
}

// 3-bit Lloyd-Max encoding of one V row spread over the wave (RowLayout
// lanes; head_dim 128 or 256, lloyd_block 128): per-128 block L2 norm (fp32
// squares summed by a pairwise tree over neighbours -- butterflies 1..32 on
// each half, then the two halves -- correctly rounded sqrt), u = v / norm (0 for a zero norm), code = first index minimising
// |u - c_j| in fp32, bit-plane words (word 3g+b holds bit b of the codes of
// elements 32g..32g+31, element 32g+i at bit i).  Lane w < 3D/32 gets word w,
// lane nb < D/128 gets norm nb.
// The per-128 block L2 norms of a V row in RowLayout lanes (head_dim 128 or
// 256): every lane gets every norm.
template <int D>
__device__ __forceinline__ void lloyd3_block_norms(const float (&x)[RowLayout<D>::E], float (&norm)[D / 128]) {
#pragma unroll
  for (int nb = 0; nb < D / 128; ++nb) {
    // Block nb holds elements 128nb + {lane, lane+64}: the tree's levels
    // h = 1 .. 32 are butterflies within each half (lane l gets its group's
    // two partial sums added in either order -- the same fp32 value), h = 64
    // adds the halves -- the order the CPU restatement uses.
    float s0 = x[2 * nb] * x[2 * nb], s1 = x[2 * nb + 1] * x[2 * nb + 1];
#pragma unroll
    for (int m = 1; m <= 32; m <<= 1) {
      s0 = s0 + shfl_xor_f(s0, m);
      s1 = s1 + shfl_xor_f(s1, m);
    }
    norm[nb] = __builtin_sqrtf(s0 + s1);
  }
}

// The lane's 3-bit codes: u = v / norm of its block (0 for a zero norm),
// code = first index minimising |u - c_j| in fp32 (sequential scan).
template <int D>
__device__ __forceinline__ void lloyd3_codes(const float (&x)[RowLayout<D>::E], const float (&norm)[D / 128],
                                             const float (&cb)[8], uint32_t (&codes)[RowLayout<D>::E]) {
#pragma unroll
  for (int j = 0; j < RowLayout<D>::E; ++j) {
    const float nrm = norm[j / 2];
    const float u = nrm > 0.0f ? x[j] / nrm : 0.0f;
    float best = fabsf(u - cb[0]);
    uint32_t c = 0;
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      float d = fabsf(u - cb[i]);
      if (d < best) {
        best = d;
        c = (uint32_t)i;
      }
    }
    codes[j] = c;
  }
}

template <int D>
__device__ __forceinline__ void lloydmax3_encode_row(const float (&x)[RowLayout<D>::E], const float (&cb)[8], int lane,
                                                      uint32_t& word_out, float& norm_out) {
  constexpr int E = RowLayout<D>::E;
  constexpr int NB = D / 128;
  constexpr int WORDS = D / 32 * 3;
  float norm[NB];
  lloyd3_block_norms<D>(x, norm);
  uint32_t codes[E];
  lloyd3_codes<D>(x, norm, cb, codes);
  // Bit-plane packing: element group g (32 elements) -> words 3g+b, bit i of
  // word 3g+b = bit b of the code of element 32g+i.  Slot j of lanes 0..31
  // is group 2j, of lanes 32..63 group 2j+1.
  uint32_t words[WORDS];
#pragma unroll
  for (int j = 0; j < E; ++j) {
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      uint64_t m = __ballot((codes[j] >> b) & 1u);
      words[3 * (2 * j) + b] = (uint32_t)m;
      words[3 * (2 * j + 1) + b] = (uint32_t)(m >> 32);
    }
  }
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < WORDS; ++i) w = (lane == i) ? words[i] : w;
  float nv = norm[0];
#pragma unroll
  for (int nb = 1; nb < NB; ++nb) nv = (lane == nb) ? norm[nb] : nv;
  word_out = w;
  norm_out = nv;
}

// Spread the low 4 bits of x into bit 0 of each byte.
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
  return ((x & 0xFu) * 0x00204081u) & 0x01010101u;
}

// fp16 lookup of 4 three-bit codes held as bytes of `sel` through byte tables
// (lo / hi bytes of the 8 fp16 codebook entries: entries 0..3 and 4..7).
__device__ __forceinline__ u32x2_t codebook_lookup4(uint32_t sel, uint32_t lo03, uint32_t lo47, uint32_t hi03,
                                                    uint32_t hi47) {
  const uint32_t lo = __builtin_amdgcn_perm(lo47, lo03, sel);
  const uint32_t hi = __builtin_amdgcn_perm(hi47, hi03, sel);
  u32x2_t r;
  r.x = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
  r.y = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
  return r;
}

}  // namespace s8kv

// Arrival at a counter word shared by the workgroups that each stored one
// partial of the same output: add `units` to the word; true for the arrival
// that completes `total` units, which also writes the word back to zero.  The
// word holds this launch's 40-bit tag above a 24-bit count; a word with
// another tag counts as zero.  Every failed
// exchange means another segment's add went in, so the loop ends.
__device__ __forceinline__ bool arrive(unsigned long long* cp, unsigned long long tag, uint32_t units, uint32_t total) {
  unsigned long long old = __hip_atomic_load(cp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    const uint32_t done = (old >> 24) == tag ? (uint32_t)(old & 0xFFFFFFu) : 0u;
    const uint32_t now = done + units;
    const unsigned long long nw = now == total ? 0ull : (tag << 24) | now;
    if (__hip_atomic_compare_exchange_weak(cp, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT))
      return now == total;
  }
}
// Agent-scope (coherence point, L2-bypassing) float store and load.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

