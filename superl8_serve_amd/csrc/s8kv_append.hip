// Paged KV append: quantize-on-write of fp16 K/V into the int8 and K8V3 layouts.
//
// One wave64 handles one (token, kv-head) row: it reads D fp16 K and V values,
// rotates K with a fixed-order fp32 Walsh-Hadamard transform, quantizes, and
// scatters the bytes to storage row (block*Hkv + h)*bs + offset.  Lane l holds
// elements l, l+64, l+128, ... so that every global access of the wave is one
// contiguous span.
#include "s8kv_device.h"
#include "s8kv_host.h"

namespace s8kv {

constexpr int kAppendWaves = 4;  // waves per workgroup

// Where a row's bytes go: through the tensor's buffer descriptor at a 32-bit
// offset (per-layer tensors up to 4 GiB), or through a 64-bit pointer (the
// <.., BIG> kernels, a tensor past 4 GiB; rows are checked against the pool
// before any store).  `off` is relative to the row's first byte.
struct BufOut {
  rsrc_t r;
  uint32_t base;
  __device__ void st128(uint32_t off, u32x4_t v) const { bstore128(v, r, base + off); }
  __device__ void st32(uint32_t off, uint32_t v) const { bstore32(v, r, base + off); }
  __device__ void st8(uint32_t off, uint8_t v) const { bstore8(v, r, base + off); }
};
struct PtrOut {
  char* p;
  __device__ void st128(uint32_t off, u32x4_t v) const { *reinterpret_cast<u32x4_t*>(p + off) = v; }
  __device__ void st32(uint32_t off, uint32_t v) const { *reinterpret_cast<uint32_t*>(p + off) = v; }
  __device__ void st8(uint32_t off, uint8_t v) const { p[off] = (char)v; }
};
template <bool BIG>
__device__ __forceinline__ auto row_out(void* base, uint32_t bytes, uint64_t off) {
  if constexpr (BIG)
    return PtrOut{static_cast<char*>(base) + off};
  else
    return BufOut{make_rsrc(base, bytes), (uint32_t)off};
}

// Per-row RTN int8 of the wave's row; writes D bytes at `byte_off` and the scale.
template <int D, class QOut, class SOut>
__device__ __forceinline__ void rtn_store_row(const float (&y)[RowLayout<D>::E], int lane, const QOut& qout,
                                              const SOut& sout) {
  constexpr int E = RowLayout<D>::E;
  int q[E];
  const float scale = rtn_row<D>(y, q);
  if (lane < RowLayout<D>::ACTIVE) {
#pragma unroll
    for (int j = 0; j < E; ++j) qout.st8((uint32_t)(lane + 64 * j), (uint8_t)(int8_t)q[j]);
  }
  if (lane == 0) sout.st32(0u, __builtin_bit_cast(uint32_t, scale));
}

struct AppendArgs {
  const _Float16* k;
  const _Float16* v;
  int64_t num_tokens;
  int num_kv_heads;
  int64_t k_stride_t, k_stride_h, v_stride_t, v_stride_h;
  const int32_t* slot_mapping;
  void* k_cache;
  void* k_scale;
  void* v_cache;   // int8 V (int8 layout) or int32 packed V (k8v3)
  void* v_scale;   // fp32 V scale (int8) or fp32 V norms (k8v3)
  const float* v_codebook;
  uint32_t kc_bytes, ks_bytes, vc_bytes, vs_bytes;
  int big;  // a tensor past 4 GiB: the <.., BIG> kernels store through 64-bit pointers
  int64_t num_blocks;
  int block_size_log2;
  float rot_norm;  // float32(1/sqrt(D))
};

template <int D, bool K8V3, bool BIG>
__global__ __launch_bounds__(64 * kAppendWaves) void append_kernel(AppendArgs a) {
  constexpr int E = RowLayout<D>::E;
  const int lane = threadIdx.x & 63;
  const int64_t row_id = (int64_t)blockIdx.x * kAppendWaves + (threadIdx.x >> 6);
  const int64_t total = a.num_tokens * a.num_kv_heads;
  if (row_id >= total) return;
  const int64_t t = row_id / a.num_kv_heads;
  const int h = (int)(row_id - t * a.num_kv_heads);
  const int32_t slot = a.slot_mapping[t];
  if (slot < 0) return;
  const int bs = 1 << a.block_size_log2;
  const uint32_t blk = (uint32_t)slot >> a.block_size_log2;
  if ((int64_t)blk >= a.num_blocks) return;  // slot outside the pool
  const uint32_t off = (uint32_t)slot & (uint32_t)(bs - 1);
  const uint32_t row = ((blk * (uint32_t)a.num_kv_heads + (uint32_t)h) << a.block_size_log2) + off;

  // both rows' loads in flight together
  float x[E], y[E];
  load_row_f16<D>(a.k + t * a.k_stride_t + h * a.k_stride_h, x, lane);
  load_row_f16<D>(a.v + t * a.v_stride_t + h * a.v_stride_h, y, lane);

  // ---- K: rotate (fp32 FWHT, one multiply, RNE to fp16) then RTN ----
  fwht_row<D>(x, lane);
#pragma unroll
  for (int j = 0; j < E; ++j) x[j] = (float)(_Float16)materialize(x[j] * a.rot_norm);
  rtn_store_row<D>(x, lane, row_out<BIG>(a.k_cache, a.kc_bytes, (uint64_t)row * D),
                   row_out<BIG>(a.k_scale, a.ks_bytes, (uint64_t)row * 4u));

  // ---- V ----
  if constexpr (!K8V3) {
    rtn_store_row<D>(y, lane, row_out<BIG>(a.v_cache, a.vc_bytes, (uint64_t)row * D),
                     row_out<BIG>(a.v_scale, a.vs_bytes, (uint64_t)row * 4u));
  } else {
    static_assert(D == 128 || D == 256, "K8V3 needs head_dim 128 or 256");
    constexpr int NB = D / 128;   // Lloyd-Max blocks per row (lloyd_block = 128)
    constexpr int WORDS = D / 32 * 3;
    float cb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cb[i] = a.v_codebook[i];
    uint32_t w;
    float nv;
    lloydmax3_encode_row<D>(y, cb, lane, w, nv);
    if (lane < WORDS) row_out<BIG>(a.v_cache, a.vc_bytes, (uint64_t)row * (WORDS * 4)).st32(lane * 4u, w);
    if (lane < NB)
      row_out<BIG>(a.v_scale, a.vs_bytes, (uint64_t)row * (NB * 4)).st32(lane * 4u, __builtin_bit_cast(uint32_t, nv));
  }
}

// int8 append with several rows per wave: a row's D values sit on LPR = D/16
// lanes, 16 consecutive values per lane, so each lane moves a row part with
// two 16-byte loads and one 16-byte store per tensor and the per-row work
// (slot lookup, addresses, reductions) is shared by 64/LPR rows per
// instruction.  The K rotation runs the FWHT stages h = 1, 2, 4, 8 in-lane
// and h = 16 .. D/2 across the row's lanes: the stage order and arithmetic of
// fwht_row, so the bytes equal the one-row-per-wave kernel's.  Needs 16-byte
// aligned K and V rows.
//
// Lane placement: part li (values 16 li .. 16 li + 15) of a row.  At head_dim
// 128 li sits on lane bits (b3 b1 b0) and lane bits (b5 b4 b2) number the row,
// so the partners of the three cross-lane stages (li ^ 1, ^ 2, ^ 4) are lanes
// ^ 1, ^ 2, ^ 8, all DPP sources.  Other head dims: li = lane % LPR.
template <int D>
struct RowsLayout {
  static constexpr int LPR = D / 16;   // lanes per row
  static constexpr int RPW = 64 / LPR;  // rows per wave
  static constexpr int LANE4 = D == 128 ? 8 : 4;  // lane xor of part xor 4
  static __device__ __forceinline__ int part(int lane) {
    return D == 128 ? (lane & 3) | ((lane >> 1) & 4) : lane % LPR;
  }
  static __device__ __forceinline__ int row(int lane) {
    return D == 128 ? ((lane >> 2) & 1) | ((lane >> 3) & 6) : lane / LPR;
  }
};

// max over the row's lanes (part xor 1, 2, 4, 8)
template <int D>
__device__ __forceinline__ float rows_max(float v) {
  constexpr int LPR = D / 16;
  if constexpr (LPR > 1) v = fmaxf(v, xor_partner<1>(v));
  if constexpr (LPR > 2) v = fmaxf(v, xor_partner<2>(v));
  if constexpr (LPR > 4) v = fmaxf(v, xor_partner<RowsLayout<D>::LANE4>(v));
  if constexpr (LPR > 8) v = fmaxf(v, xor_partner<8>(v));
  return v;
}

#define S8KV_FMAC_DPP16(CTRL)                                                         \
  "s_nop 1\n"                                                                         \
  "v_fmac_f32_dpp %0, %0, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %1, %1, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %2, %2, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %3, %3, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %4, %4, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %5, %5, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %6, %6, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %7, %7, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %8, %8, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %9, %9, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                  \
  "v_fmac_f32_dpp %10, %10, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                \
  "v_fmac_f32_dpp %11, %11, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                \
  "v_fmac_f32_dpp %12, %12, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                \
  "v_fmac_f32_dpp %13, %13, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                \
  "v_fmac_f32_dpp %14, %14, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                \
  "v_fmac_f32_dpp %15, %15, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"                \
  "s_nop 1"

// One cross-lane FWHT stage over the lane's 16 values, sign-tracked: z += t *
// (z of lane ^ M), t = -1 on the lanes whose part has the stage's bit set,
// else +1.  The lanes hold sigma * (true values), sigma = (-1)^(number of
// earlier stage bits set in the part); partners share sigma, so this is the
// butterfly on the true values (low lane a + b, high lane a - b) with the
// high lanes' sign flipped: RN(b - a) = -RN(a - b), and signed zeros aside
// (a zero quantizes to code 0 either way) the values are the untracked
// form's.  M = 1, 2, 8: one v_fmac_f32 with a DPP source per value (the s_nop
// pairs cover the DPP read-after-VALU-write hazard at the block's edges);
// M = 4 reads the partner through the LDS swizzle.
template <int M>
__device__ __forceinline__ void fwht_stage_tracked(float (&z)[16], float t) {
  if constexpr (M == 4) {
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = __builtin_fmaf(xor_partner<4>(z[i]), t, z[i]);
  } else {
    static_assert(M == 1 || M == 2 || M == 8, "DPP partners: lane ^ 1, ^ 2, ^ 8");
#define S8KV_FMAC_OPERANDS                                                                                       \
  : "+v"(z[0]), "+v"(z[1]), "+v"(z[2]), "+v"(z[3]), "+v"(z[4]), "+v"(z[5]), "+v"(z[6]), "+v"(z[7]), "+v"(z[8]), \
    "+v"(z[9]), "+v"(z[10]), "+v"(z[11]), "+v"(z[12]), "+v"(z[13]), "+v"(z[14]), "+v"(z[15])                    \
  : "v"(t)
    if constexpr (M == 1) asm(S8KV_FMAC_DPP16("quad_perm:[1,0,3,2]") S8KV_FMAC_OPERANDS);
    else if constexpr (M == 2) asm(S8KV_FMAC_DPP16("quad_perm:[2,3,0,1]") S8KV_FMAC_OPERANDS);
    else asm(S8KV_FMAC_DPP16("row_ror:8") S8KV_FMAC_OPERANDS);
#undef S8KV_FMAC_OPERANDS
  }
}
#undef S8KV_FMAC_DPP16

template <int D, class QOut, class SOut>
__device__ __forceinline__ void rows_rtn_store(const float (&y)[16], bool live, int li, const QOut& qout,
                                               const SOut& sout) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(y[i]));
  amax = rows_max<D>(amax);
  const float scale = amax / 127.0f;
  const float rscale = rtn_rscale(scale);
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    w[k] = pack_low_bytes(rtn_i8_biased(y[4 * k], scale, rscale), rtn_i8_biased(y[4 * k + 1], scale, rscale),
                          rtn_i8_biased(y[4 * k + 2], scale, rscale), rtn_i8_biased(y[4 * k + 3], scale, rscale));
  }
  if (live) {
    qout.st128((uint32_t)li * 16u, u32x4_t{w[0], w[1], w[2], w[3]});
    if (li == 0) sout.st32(0u, __builtin_bit_cast(uint32_t, scale));
  }
}

// 2 w + b in one add with carry-in (the lanes' b as a wave mask).
__device__ __forceinline__ uint32_t shift_in_bit(uint32_t w, bool b) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(b);
  uint32_t r;
  uint64_t carry_out;
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(carry_out) : "v"(w), "s"(m));
  return r;
}

// Ordered key of an fp32 bit pattern: key(x) < key(y) iff x < y, with -0
// just below +0; the map is its own inverse.
__device__ __forceinline__ int f32_key(int bits) { return bits ^ ((bits >> 31) & 0x7FFFFFFF); }

// Threshold T of the codebook neighbours a = c_{j-1} < b = c_j: the least
// fp32 u for which entry j is strictly nearer than entry j - 1 (fabsf(u - b) <
// fabsf(u - a), lloyd3_search's test).  On [a, b] the two distances are
// RN(b - u), non-increasing in u, and RN(u - a), non-decreasing, so the test
// is monotone there -- false at a, true at b -- and bisection over the keys
// finds T.  Below a the test is false (RN(b - u) >= RN(a - u)) and above b,
// for a codebook accepted by lloyd3_search_ok and |u| <= 1, true; so for
// every u the encoder sees, the test equals u >= T.  (T is never +0: -0 gives
// the same distances and precedes it.)
__device__ __forceinline__ float lloyd3_threshold(float a, float b) {
  int lo = f32_key(__builtin_bit_cast(int, a)), hi = f32_key(__builtin_bit_cast(int, b));
  for (int it = 0; it < 32; ++it) {
    const uint32_t d = (uint32_t)hi - (uint32_t)lo;
    if (d <= 1u) break;
    const int mid = (int)((uint32_t)lo + (d >> 1));
    const float u = __builtin_bit_cast(float, f32_key(mid));
    if (fabsf(u - b) < fabsf(u - a)) hi = mid;
    else lo = mid;
  }
  return __builtin_bit_cast(float, f32_key(hi));
}

// 3-bit Lloyd-Max V of the lane's 16 values (head_dim 128 or 256, blocks of
// 128 = 8 lanes): the block's L2 norm adds the fp32 squares in the order of
// lloydmax3_encode_row (a pairwise tree over neighbours: levels h = 1 .. 8
// in-lane, h = 16, 32, 64 across the parts ^ 1, ^ 2, ^ 4), correctly rounded
// sqrt; u = v / norm (0 for a zero norm) as the Markstein quotient from the
// block's reciprocal, which equals the IEEE quotient for an fp16 v and any
// fp32 norm (checked for every pair of significands); code = first index
// minimising |u - c_j|: with `search` (a codebook accepted by
// lloyd3_search_ok) lloyd3_search's three tests as compares against the
// thresholds thr[j] = T_j, else the sequential scan.  Parts 2g and 2g + 1
// (lanes l and l ^ 1) hold elements 32g .. 32g + 31: each builds 16 bits of
// the three bit-plane words 3g + b, and the even part stores them.
template <int D, class VOut, class NOut>
__device__ __forceinline__ void rows_lloydmax3_store(const float (&x)[16], bool live, int li, bool search,
                                                     const float (&cb)[8], const float (&thr)[8], const VOut& vout,
                                                     const NOut& nout) {
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = x[i] * x[i];
#pragma unroll
  for (int h = 1; h < 16; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 16; i += 2 * h) s[i] = s[i] + s[i + h];
  }
  float t = s[0];  // the lane's 16 elements; partners hold the neighbouring groups
  t = t + xor_partner<1>(t);
  t = t + xor_partner<2>(t);
  t = t + xor_partner<RowsLayout<D>::LANE4>(t);
  const float nrm = __builtin_sqrtf(t);
  const float rn = rtn_rscale(nrm);  // 1 / norm, 0 for a zero norm (then u = 0)
  float u[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float q0 = materialize(x[i] * rn);
    const float r = __builtin_fmaf(-q0, nrm, x[i]);
    u[i] = __builtin_fmaf(r, rn, q0);
  }
  // bit i of pw[b] = bit b of element i's code (elements shifted in from 15 down)
  uint32_t pw[3] = {0u, 0u, 0u};
  if (search) {
#pragma unroll
    for (int i = 15; i >= 0; --i) {
      const bool b2 = u[i] >= thr[4];
      const bool b1 = u[i] >= (b2 ? thr[6] : thr[2]);
      const float t_hi = b2 ? thr[7] : thr[3], t_lo = b2 ? thr[5] : thr[1];
      const bool b0 = u[i] >= (b1 ? t_hi : t_lo);
      pw[0] = shift_in_bit(pw[0], b0);
      pw[1] = shift_in_bit(pw[1], b1);
      pw[2] = shift_in_bit(pw[2], b2);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float best = fabsf(u[i] - cb[0]);
      uint32_t c = 0;
#pragma unroll
      for (int j = 1; j < 8; ++j) {
        const float d = fabsf(u[i] - cb[j]);
        if (d < best) {
          best = d;
          c = (uint32_t)j;
        }
      }
#pragma unroll
      for (int b = 0; b < 3; ++b) pw[b] |= ((c >> b) & 1u) << i;
    }
  }
  uint32_t w[3];
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const uint32_t odd = (uint32_t)__builtin_amdgcn_mov_dpp((int)pw[b], 0xB1, 0xF, 0xF, false);  // lane ^ 1
    w[b] = pw[b] | (odd << 16);
  }
  if (live && (li & 1) == 0) {
#pragma unroll
    for (int b = 0; b < 3; ++b) vout.st32((uint32_t)(li / 2) * 12u + 4u * b, w[b]);
  }
  if (live && (li & 7) == 0) nout.st32((uint32_t)(li / 8) * 4u, __builtin_bit_cast(uint32_t, nrm));
}

// Row groups (kAppendWaves waves of RPW rows) per workgroup: the K8V3 kernel
// derives the codebook's thresholds once per workgroup and reuses them.
template <bool K8V3>
constexpr int kRowsIters = K8V3 ? 4 : 1;

template <int D, bool K8V3, bool BIG>
__global__ __launch_bounds__(64 * kAppendWaves) void append_rows_kernel(AppendArgs a) {
  using L = RowsLayout<D>;
  constexpr int LPR = L::LPR;
  constexpr int RPW = L::RPW;
  const int lane = threadIdx.x & 63;
  const int li = L::part(lane);
  // FWHT sign tracking: the stage multipliers of the lane, and the lane's
  // final sign (-1)^popcount(li) folded into the 1/sqrt(D) multiply
  const float t1 = (li & 1) ? -1.0f : 1.0f, t2 = (li & 2) ? -1.0f : 1.0f;
  const float t4 = (li & 4) ? -1.0f : 1.0f, t8 = (li & 8) ? -1.0f : 1.0f;
  const float srn = (__builtin_popcount(li) & 1) ? -a.rot_norm : a.rot_norm;

  float cb[8], thr[8];
  bool search = false;
  if constexpr (K8V3) {
    __shared__ float thr_lds[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cb[i] = a.v_codebook[i];
    search = lloyd3_search_ok(cb);  // uniform over the workgroup
    if (search) {
      if (threadIdx.x < 7) thr_lds[threadIdx.x + 1] = lloyd3_threshold(a.v_codebook[threadIdx.x], a.v_codebook[threadIdx.x + 1]);
      __syncthreads();
#pragma unroll
      for (int j = 1; j < 8; ++j) thr[j] = thr_lds[j];
    }
    thr[0] = 0.0f;
  }

  const int64_t total = a.num_tokens * a.num_kv_heads;
#pragma unroll 1
  for (int it = 0; it < kRowsIters<K8V3>; ++it) {
    const int64_t row_id =
        (((int64_t)blockIdx.x * kRowsIters<K8V3> + it) * kAppendWaves + (threadIdx.x >> 6)) * RPW + L::row(lane);
    bool live = row_id < total;
    int64_t t = 0;
    int h = 0;
    uint32_t row = 0;
    if (live) {
      t = row_id / a.num_kv_heads;
      h = (int)(row_id - t * a.num_kv_heads);
      const int32_t slot = a.slot_mapping[t];
      const uint32_t blk = (uint32_t)slot >> a.block_size_log2;
      live = slot >= 0 && (int64_t)blk < a.num_blocks;  // negative slots and slots outside the pool are skipped
      row = ((blk * (uint32_t)a.num_kv_heads + (uint32_t)h) << a.block_size_log2) +
            ((uint32_t)slot & ((1u << a.block_size_log2) - 1u));
    }
    // both row parts' loads in flight together
    float x[16], y[16];
    {
      half8_t k0{}, k1{}, v0{}, v1{};
      if (live) {
        const _Float16* kp = a.k + t * a.k_stride_t + h * a.k_stride_h + li * 16;
        const _Float16* vp = a.v + t * a.v_stride_t + h * a.v_stride_h + li * 16;
        k0 = *reinterpret_cast<const half8_t*>(kp);
        k1 = *reinterpret_cast<const half8_t*>(kp + 8);
        v0 = *reinterpret_cast<const half8_t*>(vp);
        v1 = *reinterpret_cast<const half8_t*>(vp + 8);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[i] = (float)k0[i];
        x[8 + i] = (float)k1[i];
        y[i] = (float)v0[i];
        y[8 + i] = (float)v1[i];
      }
    }

    // ---- K: rotate (fp32 FWHT, one multiply, RNE to fp16) then RTN ----
#pragma unroll
    for (int hs = 1; hs < 16; hs <<= 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if ((i & hs) == 0) {
          const float p0 = x[i], p1 = x[i + hs];
          x[i] = p0 + p1;
          x[i + hs] = p0 - p1;
        }
      }
    }
    if constexpr (LPR > 1) fwht_stage_tracked<1>(x, t1);
    if constexpr (LPR > 2) fwht_stage_tracked<2>(x, t2);
    if constexpr (LPR > 4) fwht_stage_tracked<L::LANE4>(x, t4);
    if constexpr (LPR > 8) fwht_stage_tracked<8>(x, t8);
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (float)(_Float16)materialize(x[i] * srn);
    rows_rtn_store<D>(x, live, li, row_out<BIG>(a.k_cache, a.kc_bytes, (uint64_t)row * D),
                      row_out<BIG>(a.k_scale, a.ks_bytes, (uint64_t)row * 4u));

    // ---- V: RTN, or 3-bit Lloyd-Max ----
    if constexpr (!K8V3) {
      rows_rtn_store<D>(y, live, li, row_out<BIG>(a.v_cache, a.vc_bytes, (uint64_t)row * D),
                        row_out<BIG>(a.v_scale, a.vs_bytes, (uint64_t)row * 4u));
    } else {
      static_assert(D == 128 || D == 256, "K8V3 needs head_dim 128 or 256");
      rows_lloydmax3_store<D>(y, live, li, search, cb, thr,
                              row_out<BIG>(a.v_cache, a.vc_bytes, (uint64_t)row * (D / 32 * 3 * 4)),
                              row_out<BIG>(a.v_scale, a.vs_bytes, (uint64_t)row * (D / 128 * 4)));
    }
  }
}

template <bool K8V3, bool BIG>
static int launch_append_impl(const AppendArgs& a, int head_dim, hipStream_t stream) {
  const int64_t rows = a.num_tokens * a.num_kv_heads;
  if (rows == 0) return S8KV_OK;
  const bool rows16 = ((uintptr_t)a.k % 16 == 0) && ((uintptr_t)a.v % 16 == 0) && a.k_stride_t % 8 == 0 &&
                      a.k_stride_h % 8 == 0 && a.v_stride_t % 8 == 0 && a.v_stride_h % 8 == 0;
  if (rows16) {  // several rows per wave
    const int rows_per_wg = kAppendWaves * 64 / (head_dim / 16) * kRowsIters<K8V3>;
    const int64_t grid = (rows + rows_per_wg - 1) / rows_per_wg;
    S8KV_REQUIRE(grid < (int64_t(1) << 31), S8KV_ERR_INVALID, "append: too many rows (%lld)", (long long)rows);
    dim3 g((unsigned)grid), b(64 * kAppendWaves);
    switch (head_dim) {
      case 32:
        if constexpr (!K8V3) { hipLaunchKernelGGL((append_rows_kernel<32, false, BIG>), g, b, 0, stream, a); break; }
        return S8KV_ERR_UNSUPPORTED;
      case 64:
        if constexpr (!K8V3) { hipLaunchKernelGGL((append_rows_kernel<64, false, BIG>), g, b, 0, stream, a); break; }
        return S8KV_ERR_UNSUPPORTED;
      case 128: hipLaunchKernelGGL((append_rows_kernel<128, K8V3, BIG>), g, b, 0, stream, a); break;
      case 256: hipLaunchKernelGGL((append_rows_kernel<256, K8V3, BIG>), g, b, 0, stream, a); break;
      default: return S8KV_ERR_UNSUPPORTED;
    }
    return check_launch(K8V3 ? "s8kv_append_k8v3" : "s8kv_append_int8");
  }
  const int64_t grid = (rows + kAppendWaves - 1) / kAppendWaves;
  S8KV_REQUIRE(grid < (int64_t(1) << 31), S8KV_ERR_INVALID, "append: too many rows (%lld)", (long long)rows);
  dim3 g((unsigned)grid), b(64 * kAppendWaves);
  switch (head_dim) {
    case 32:
      if constexpr (!K8V3) { hipLaunchKernelGGL((append_kernel<32, false, BIG>), g, b, 0, stream, a); break; }
      return S8KV_ERR_UNSUPPORTED;
    case 64:
      if constexpr (!K8V3) { hipLaunchKernelGGL((append_kernel<64, false, BIG>), g, b, 0, stream, a); break; }
      return S8KV_ERR_UNSUPPORTED;
    case 128: hipLaunchKernelGGL((append_kernel<128, K8V3, BIG>), g, b, 0, stream, a); break;
    case 256: hipLaunchKernelGGL((append_kernel<256, K8V3, BIG>), g, b, 0, stream, a); break;
    default: return S8KV_ERR_UNSUPPORTED;
  }
  return check_launch(K8V3 ? "s8kv_append_k8v3" : "s8kv_append_int8");
}

template <bool K8V3>
static int launch_append(const AppendArgs& a, int head_dim, hipStream_t stream) {
  return a.big ? launch_append_impl<K8V3, true>(a, head_dim, stream) : launch_append_impl<K8V3, false>(a, head_dim, stream);
}

static int common_append_checks(const void* k, const void* v, int64_t num_tokens, int num_kv_heads, int head_dim,
                                const int32_t* slot_mapping, int64_t num_blocks, int block_size) {
  S8KV_REQUIRE(num_tokens >= 0, S8KV_ERR_INVALID, "append: num_tokens < 0");
  S8KV_REQUIRE(num_kv_heads > 0, S8KV_ERR_INVALID, "append: num_kv_heads must be > 0");
  S8KV_REQUIRE(head_dim_ok(head_dim), S8KV_ERR_UNSUPPORTED, "append: head_dim %d not in {32,64,128,256}", head_dim);
  S8KV_REQUIRE(is_pow2(block_size) && block_size >= 4, S8KV_ERR_UNSUPPORTED,
               "append: block_size %d must be a power of two >= 4", block_size);
  S8KV_REQUIRE(num_blocks > 0, S8KV_ERR_INVALID, "append: num_blocks must be > 0");
  S8KV_REQUIRE(num_tokens == 0 || (k && v && slot_mapping), S8KV_ERR_INVALID, "append: null input pointer");
  return S8KV_OK;
}

}  // namespace s8kv

using namespace s8kv;

extern "C" int s8kv_append_int8(const void* k, const void* v, int64_t num_tokens, int num_kv_heads, int head_dim,
                                int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h,
                                const int32_t* slot_mapping, int8_t* k_cache, float* k_scale, int8_t* v_cache,
                                float* v_scale, int64_t num_blocks, int block_size, void* stream) {
  int rc = common_append_checks(k, v, num_tokens, num_kv_heads, head_dim, slot_mapping, num_blocks, block_size);
  if (rc) return rc;
  const int64_t rows = num_blocks * num_kv_heads * block_size;
  S8KV_REQUIRE(fits_u32(rows), S8KV_ERR_UNSUPPORTED, "append: more than 2^32 cache rows per layer");
  S8KV_REQUIRE(k_cache && k_scale && v_cache && v_scale, S8KV_ERR_INVALID, "append: null cache pointer");
  AppendArgs a{};
  a.k = (const _Float16*)k;
  a.v = (const _Float16*)v;
  a.num_tokens = num_tokens;
  a.num_kv_heads = num_kv_heads;
  a.k_stride_t = k_stride_t; a.k_stride_h = k_stride_h;
  a.v_stride_t = v_stride_t; a.v_stride_h = v_stride_h;
  a.slot_mapping = slot_mapping;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_cache; a.v_scale = v_scale;
  a.big = !fits_u32(rows * head_dim);
  a.kc_bytes = cap_u32((uint64_t)(rows * head_dim));
  a.vc_bytes = cap_u32((uint64_t)(rows * head_dim));
  a.ks_bytes = cap_u32((uint64_t)(rows * 4));
  a.vs_bytes = cap_u32((uint64_t)(rows * 4));
  a.num_blocks = num_blocks;
  a.block_size_log2 = log2i(block_size);
  a.rot_norm = (float)(1.0 / __builtin_sqrt((double)head_dim));
  return launch_append<false>(a, head_dim, (hipStream_t)stream);
}

extern "C" int s8kv_append_k8v3(const void* k, const void* v, int64_t num_tokens, int num_kv_heads, int head_dim,
                                int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h,
                                const int32_t* slot_mapping, int8_t* k_cache, float* k_scale, int32_t* v_packed,
                                float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                                int block_size, void* stream) {
  int rc = common_append_checks(k, v, num_tokens, num_kv_heads, head_dim, slot_mapping, num_blocks, block_size);
  if (rc) return rc;
  S8KV_REQUIRE(head_dim == 128 || head_dim == 256, S8KV_ERR_UNSUPPORTED,
               "append_k8v3: head_dim %d not in {128, 256}", head_dim);
  S8KV_REQUIRE(lloyd_block == 128, S8KV_ERR_UNSUPPORTED, "append_k8v3: lloyd_block %d != 128", lloyd_block);
  S8KV_REQUIRE(k_cache && k_scale && v_packed && v_norm && v_codebook, S8KV_ERR_INVALID,
               "append_k8v3: null cache pointer");
  const int64_t rows = num_blocks * num_kv_heads * block_size;
  S8KV_REQUIRE(fits_u32(rows), S8KV_ERR_UNSUPPORTED, "append_k8v3: more than 2^32 cache rows per layer");
  AppendArgs a{};
  a.k = (const _Float16*)k;
  a.v = (const _Float16*)v;
  a.num_tokens = num_tokens;
  a.num_kv_heads = num_kv_heads;
  a.k_stride_t = k_stride_t; a.k_stride_h = k_stride_h;
  a.v_stride_t = v_stride_t; a.v_stride_h = v_stride_h;
  a.slot_mapping = slot_mapping;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_packed; a.v_scale = v_norm;
  a.v_codebook = v_codebook;
  a.big = !fits_u32(rows * head_dim);
  a.kc_bytes = cap_u32((uint64_t)(rows * head_dim));
  a.ks_bytes = cap_u32((uint64_t)(rows * 4));
  a.vc_bytes = cap_u32((uint64_t)(rows * (head_dim / 32 * 3) * 4));
  a.vs_bytes = cap_u32((uint64_t)(rows * (head_dim / 128) * 4));
  a.num_blocks = num_blocks;
  a.block_size_log2 = log2i(block_size);
  a.rot_norm = (float)(1.0 / __builtin_sqrt((double)head_dim));
  return launch_append<true>(a, head_dim, (hipStream_t)stream);
}
