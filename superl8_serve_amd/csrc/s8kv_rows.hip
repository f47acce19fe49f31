// Row-wise codec kernels behind the helper functions the reference's cache
// code calls on its `superl8` module (rotate_last, quantize_i8_rowwise,
// quantize_lloydmax, pack_indices_lowbit, unpack_indices_lowbit): one wave per
// (token, head) row with the append kernel's device functions, so a row
// written through these helpers holds the bytes the fused append writes.
#include "s8kv_device.h"
#include "s8kv_host.h"

namespace s8kv {
namespace rows {

constexpr int kWaves = 4;

// fp32 -> bf16, round to nearest even (NaN -> quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// dtype codes of s8kv_rotate_rows: 0 fp16, 1 bf16, 2 fp32
template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == 0) return (float)reinterpret_cast<const _Float16*>(p)[i];
  if constexpr (DT == 1)
    return __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
  return reinterpret_cast<const float*>(p)[i];
}
template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
  if constexpr (DT == 0) reinterpret_cast<_Float16*>(p)[i] = (_Float16)v;
  else if constexpr (DT == 1) reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v);
  else reinterpret_cast<float*>(p)[i] = v;
}

// out = rotate_last(x): fp32 FWHT (the append's stage order), one fp32
// multiply by fp32(1/sqrt(D)), round to the element type.
template <int D, int DT>
__global__ __launch_bounds__(64 * kWaves) void rotate_rows_kernel(const void* x, int64_t nrows, int64_t xs, void* out,
                                                                  int64_t os, float rot_norm) {
  constexpr int E = RowLayout<D>::E;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (r >= nrows) return;
  float v[E];
#pragma unroll
  for (int j = 0; j < E; ++j) v[j] = lane < RowLayout<D>::ACTIVE ? load_elem<DT>(x, r * xs + lane + 64 * j) : 0.0f;
  fwht_row<D>(v, lane);
  if (lane < RowLayout<D>::ACTIVE) {
#pragma unroll
    for (int j = 0; j < E; ++j) store_elem<DT>(out, r * os + lane + 64 * j, materialize(v[j] * rot_norm));
  }
}

// Per-row RTN int8 of fp16 rows, optionally after rotate_last (the append's
// K path); q [nrows][D] and scale [nrows] contiguous.
template <int D>
__global__ __launch_bounds__(64 * kWaves) void quantize_rows_int8_kernel(const _Float16* x, int64_t nrows, int64_t xs,
                                                                         int rotate, float rot_norm, int8_t* q,
                                                                         float* scale) {
  constexpr int E = RowLayout<D>::E;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (r >= nrows) return;
  float v[E];
  load_row_f16<D>(x + r * xs, v, lane);
  if (rotate) {
    fwht_row<D>(v, lane);
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = (float)(_Float16)materialize(v[j] * rot_norm);
  }
  int qv[E];
  const float s = rtn_row<D>(v, qv);
  if (lane < RowLayout<D>::ACTIVE) {
#pragma unroll
    for (int j = 0; j < E; ++j) q[r * D + lane + 64 * j] = (int8_t)qv[j];
  }
  if (lane == 0) scale[r] = s;
}

// 3-bit Lloyd-Max codes (one byte per element) and per-128 block norms of
// fp16 rows: the arithmetic of the append's K8V3 V path.
template <int D>
__global__ __launch_bounds__(64 * kWaves) void lloydmax3_rows_kernel(const _Float16* v, int64_t nrows, int64_t vs,
                                                                     const float* codebook, uint8_t* codes,
                                                                     float* norms) {
  constexpr int E = RowLayout<D>::E;
  constexpr int NB = D / 128;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (r >= nrows) return;
  float cb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cb[i] = codebook[i];
  float x[E];
  load_row_f16<D>(v + r * vs, x, lane);
  float norm[NB];
  lloyd3_block_norms<D>(x, norm);
  uint32_t c[E];
  lloyd3_codes<D>(x, norm, cb, c);
#pragma unroll
  for (int j = 0; j < E; ++j) codes[r * D + lane + 64 * j] = (uint8_t)c[j];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
    if (lane == nb) norms[r * NB + nb] = norm[nb];
}

// Bit-plane packing of 3-bit codes: group g (codes 32g .. 32g+31) -> words
// 3g + b holding bit b of each code, element 32g+i at bit i.  One thread per
// group; codes are taken modulo 8.
__global__ __launch_bounds__(256) void pack3_kernel(const uint8_t* codes, int64_t ngroups, uint32_t* words) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= ngroups) return;
  const uint8_t* c = codes + i * 32;
  uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const uint32_t x = c[e];
    w0 |= (x & 1u) << e;
    w1 |= ((x >> 1) & 1u) << e;
    w2 |= ((x >> 2) & 1u) << e;
  }
  words[3 * i] = w0;
  words[3 * i + 1] = w1;
  words[3 * i + 2] = w2;
}

__global__ __launch_bounds__(256) void unpack3_kernel(const uint32_t* words, int64_t ngroups, uint8_t* codes) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= ngroups) return;
  const uint32_t w0 = words[3 * i], w1 = words[3 * i + 1], w2 = words[3 * i + 2];
  uint8_t* c = codes + i * 32;
#pragma unroll
  for (int e = 0; e < 32; ++e) c[e] = (uint8_t)(((w0 >> e) & 1u) | (((w1 >> e) & 1u) << 1) | (((w2 >> e) & 1u) << 2));
}

inline int64_t row_grid(int64_t nrows) { return (nrows + kWaves - 1) / kWaves; }

}  // namespace rows
}  // namespace s8kv

using namespace s8kv;

extern "C" int s8kv_rotate_rows(const void* x, int64_t num_rows, int head_dim, int64_t x_row_stride, int dtype,
                                void* out, int64_t out_row_stride, void* stream) {
  S8KV_REQUIRE(num_rows >= 0, S8KV_ERR_INVALID, "rotate_rows: num_rows < 0");
  S8KV_REQUIRE(head_dim_ok(head_dim), S8KV_ERR_UNSUPPORTED, "rotate_rows: head_dim %d not in {32,64,128,256}",
               head_dim);
  S8KV_REQUIRE(dtype >= 0 && dtype <= 2, S8KV_ERR_UNSUPPORTED, "rotate_rows: dtype code %d not in {0,1,2}", dtype);
  if (num_rows == 0) return S8KV_OK;
  S8KV_REQUIRE(x && out, S8KV_ERR_INVALID, "rotate_rows: null pointer argument");
  S8KV_REQUIRE(x_row_stride >= head_dim && out_row_stride >= head_dim, S8KV_ERR_INVALID,
               "rotate_rows: row strides must be >= head_dim");
  const int64_t grid = rows::row_grid(num_rows);
  S8KV_REQUIRE(grid <= INT32_MAX, S8KV_ERR_UNSUPPORTED, "rotate_rows: too many rows");
  const float rn = (float)(1.0 / __builtin_sqrt((double)head_dim));
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)grid), b(64 * rows::kWaves);
#define S8KV_ROT(D, DT) \
  hipLaunchKernelGGL((rows::rotate_rows_kernel<D, DT>), g, b, 0, s, x, num_rows, x_row_stride, out, out_row_stride, rn)
#define S8KV_ROT_D(D)            \
  switch (dtype) {               \
    case 0: S8KV_ROT(D, 0); break; \
    case 1: S8KV_ROT(D, 1); break; \
    default: S8KV_ROT(D, 2); break; \
  }
  switch (head_dim) {
    case 32: S8KV_ROT_D(32); break;
    case 64: S8KV_ROT_D(64); break;
    case 128: S8KV_ROT_D(128); break;
    default: S8KV_ROT_D(256); break;
  }
#undef S8KV_ROT_D
#undef S8KV_ROT
  return check_launch("s8kv_rotate_rows");
}

extern "C" int s8kv_quantize_rows_int8(const void* x, int64_t num_rows, int head_dim, int64_t x_row_stride,
                                       int rotate, int8_t* q, float* scale, void* stream) {
  S8KV_REQUIRE(num_rows >= 0, S8KV_ERR_INVALID, "quantize_rows_int8: num_rows < 0");
  S8KV_REQUIRE(head_dim_ok(head_dim), S8KV_ERR_UNSUPPORTED,
               "quantize_rows_int8: head_dim %d not in {32,64,128,256}", head_dim);
  if (num_rows == 0) return S8KV_OK;
  S8KV_REQUIRE(x && q && scale, S8KV_ERR_INVALID, "quantize_rows_int8: null pointer argument");
  S8KV_REQUIRE(x_row_stride >= head_dim, S8KV_ERR_INVALID, "quantize_rows_int8: row stride must be >= head_dim");
  const int64_t grid = rows::row_grid(num_rows);
  S8KV_REQUIRE(grid <= INT32_MAX, S8KV_ERR_UNSUPPORTED, "quantize_rows_int8: too many rows");
  const float rn = (float)(1.0 / __builtin_sqrt((double)head_dim));
  const _Float16* xp = (const _Float16*)x;
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)grid), b(64 * rows::kWaves);
  switch (head_dim) {
    case 32: hipLaunchKernelGGL(rows::quantize_rows_int8_kernel<32>, g, b, 0, s, xp, num_rows, x_row_stride, rotate, rn, q, scale); break;
    case 64: hipLaunchKernelGGL(rows::quantize_rows_int8_kernel<64>, g, b, 0, s, xp, num_rows, x_row_stride, rotate, rn, q, scale); break;
    case 128: hipLaunchKernelGGL(rows::quantize_rows_int8_kernel<128>, g, b, 0, s, xp, num_rows, x_row_stride, rotate, rn, q, scale); break;
    default: hipLaunchKernelGGL(rows::quantize_rows_int8_kernel<256>, g, b, 0, s, xp, num_rows, x_row_stride, rotate, rn, q, scale); break;
  }
  return check_launch("s8kv_quantize_rows_int8");
}

extern "C" int s8kv_quantize_rows_lloydmax3(const void* v, int64_t num_rows, int head_dim, int64_t v_row_stride,
                                            const float* codebook, uint8_t* codes, float* norms, void* stream) {
  S8KV_REQUIRE(num_rows >= 0, S8KV_ERR_INVALID, "quantize_rows_lloydmax3: num_rows < 0");
  S8KV_REQUIRE(head_dim == 128 || head_dim == 256, S8KV_ERR_UNSUPPORTED,
               "quantize_rows_lloydmax3: head_dim %d not in {128, 256} (lloyd_block 128)", head_dim);
  if (num_rows == 0) return S8KV_OK;
  S8KV_REQUIRE(v && codebook && codes && norms, S8KV_ERR_INVALID, "quantize_rows_lloydmax3: null pointer argument");
  S8KV_REQUIRE(v_row_stride >= head_dim, S8KV_ERR_INVALID, "quantize_rows_lloydmax3: row stride must be >= head_dim");
  const int64_t grid = rows::row_grid(num_rows);
  S8KV_REQUIRE(grid <= INT32_MAX, S8KV_ERR_UNSUPPORTED, "quantize_rows_lloydmax3: too many rows");
  const _Float16* vp = (const _Float16*)v;
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)grid), b(64 * rows::kWaves);
  if (head_dim == 128)
    hipLaunchKernelGGL(rows::lloydmax3_rows_kernel<128>, g, b, 0, s, vp, num_rows, v_row_stride, codebook, codes, norms);
  else
    hipLaunchKernelGGL(rows::lloydmax3_rows_kernel<256>, g, b, 0, s, vp, num_rows, v_row_stride, codebook, codes, norms);
  return check_launch("s8kv_quantize_rows_lloydmax3");
}

extern "C" int s8kv_pack_codes3(const uint8_t* codes, int64_t num_rows, int head_dim, int32_t* words, void* stream) {
  S8KV_REQUIRE(num_rows >= 0 && head_dim > 0 && head_dim % 32 == 0, S8KV_ERR_INVALID,
               "pack_codes3: head_dim %d must be a positive multiple of 32", head_dim);
  const int64_t groups = num_rows * (head_dim / 32);
  if (groups == 0) return S8KV_OK;
  S8KV_REQUIRE(codes && words, S8KV_ERR_INVALID, "pack_codes3: null pointer argument");
  const int64_t grid = (groups + 255) / 256;
  S8KV_REQUIRE(grid <= INT32_MAX, S8KV_ERR_UNSUPPORTED, "pack_codes3: too many rows");
  hipLaunchKernelGGL(rows::pack3_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, codes, groups,
                     reinterpret_cast<uint32_t*>(words));
  return check_launch("s8kv_pack_codes3");
}

extern "C" int s8kv_unpack_codes3(const int32_t* words, int64_t num_rows, int head_dim, uint8_t* codes,
                                  void* stream) {
  S8KV_REQUIRE(num_rows >= 0 && head_dim > 0 && head_dim % 32 == 0, S8KV_ERR_INVALID,
               "unpack_codes3: head_dim %d must be a positive multiple of 32", head_dim);
  const int64_t groups = num_rows * (head_dim / 32);
  if (groups == 0) return S8KV_OK;
  S8KV_REQUIRE(codes && words, S8KV_ERR_INVALID, "unpack_codes3: null pointer argument");
  const int64_t grid = (groups + 255) / 256;
  S8KV_REQUIRE(grid <= INT32_MAX, S8KV_ERR_UNSUPPORTED, "unpack_codes3: too many rows");
  hipLaunchKernelGGL(rows::unpack3_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint32_t*>(words), groups, codes);
  return check_launch("s8kv_unpack_codes3");
}
