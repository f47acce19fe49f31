// Prompt-time KV eviction: SnapKV attention scores of the last query over a
// sequence's keys, and the keep-list gather that moves the kept tokens'
// quantized rows into fresh blocks byte for byte.
//
// Scores (three launches): logits [Hq][n] = scale * q_h . K_t with K the
// dequantized paged int8 K (q rotated, since K is stored rotated: q . H k =
// (H q) . k) or a dense fp16 / fp32 K; then each head's max and softmax sum;
// then score_t = mean over heads of exp(logit - max) / sum.  A workgroup owns
// 64 tokens of one KV head (one token per lane) and the G q heads of its
// group (the 4 waves split them); K rows are read in 32-dim chunks.
//
// Gather: for each kept token j, every (layer, cache tensor, KV head) row at
// src_slots[j] is copied to dst_slots[j] (4-byte words).
#include "s8kv_device.h"
#include "s8kv_host.h"

namespace s8kv {
namespace evict {

constexpr int kWaves = 4;
constexpr int kTok = 64;            // tokens per workgroup
constexpr int kMaxGroupDims = 16384;  // G * D floats of q kept in LDS

struct ScoreArgs {
  const void* q;          // [Hq][D] rows at q_stride elements
  int64_t q_stride;
  int q_f32;              // q element type: 0 fp16, 1 fp32
  int num_q_heads, num_kv_heads, group, n;
  float scale;            // softmax scale
  float rot_norm;         // paged: fp32(1/sqrt(D))
  // paged int8 K (one sequence): its block ids in order
  const void* k_cache;
  const void* k_scale;
  int64_t num_blocks;
  const int32_t* block_row;
  int bs_log2;
  // dense K [Hkv][n][D]
  const void* k;
  int64_t k_stride_h, k_stride_t;
  int k_f32;
  float* logits;          // [Hq][n]
  float* stats;           // [Hq][2]: max, sum of exp(logit - max)
  float* scores;          // [n]
};

template <int D>
__device__ __forceinline__ void load_q_row(const ScoreArgs& a, int head, float (&x)[RowLayout<D>::E], int lane) {
#pragma unroll
  for (int j = 0; j < RowLayout<D>::E; ++j) {
    const int e = lane + 64 * j;
    float v = 0.0f;
    if (lane < RowLayout<D>::ACTIVE) {
      const int64_t i = (int64_t)head * a.q_stride + e;
      v = a.q_f32 ? reinterpret_cast<const float*>(a.q)[i] : (float)reinterpret_cast<const _Float16*>(a.q)[i];
    }
    x[j] = v;
  }
}

template <int D, bool PAGED>
__global__ __launch_bounds__(64 * kWaves) void snapkv_logits_kernel(ScoreArgs a) {
  extern __shared__ __attribute__((aligned(16))) float qs[];  // [G][D], scaled (and rotated when PAGED)
  constexpr int E = RowLayout<D>::E;
  const int h = blockIdx.y;
  const int G = a.group;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int g = wave; g < G; g += kWaves) {
    float x[E];
    load_q_row<D>(a, h * G + g, x, lane);
    if constexpr (PAGED) fwht_row<D>(x, lane);
    if (lane < RowLayout<D>::ACTIVE) {
#pragma unroll
      for (int j = 0; j < E; ++j) qs[g * D + lane + 64 * j] = PAGED ? x[j] * a.rot_norm * a.scale : x[j] * a.scale;
    }
  }
  __syncthreads();
  const int t = blockIdx.x * kTok + lane;
  if (t >= a.n) return;
  float kscale = 1.0f;
  const char* krow = nullptr;  // paged: the token's int8 K row (64-bit addressing: pools past 4 GiB)
  if constexpr (PAGED) {
    const uint32_t bsm = (1u << a.bs_log2) - 1u;
    const uint32_t blk = (uint32_t)a.block_row[t >> a.bs_log2];
    if ((int64_t)blk < a.num_blocks) {  // a block id outside the pool scores as a zero key
      const uint64_t row = ((uint64_t)blk * (uint32_t)a.num_kv_heads + (uint32_t)h) * (1u << a.bs_log2) +
                           ((uint32_t)t & bsm);
      kscale = reinterpret_cast<const float*>(a.k_scale)[row];
      krow = static_cast<const char*>(a.k_cache) + row * D;
    } else {
      kscale = 0.0f;
    }
  }
  constexpr int kMaxHeads = 16;  // q heads per wave: G <= 64
  float acc[kMaxHeads];
#pragma unroll
  for (int i = 0; i < kMaxHeads; ++i) acc[i] = 0.0f;
  for (int c = 0; c < D; c += 32) {
    float kv[32];
    if constexpr (PAGED) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const u32x4_t w = krow ? *reinterpret_cast<const u32x4_t*>(krow + c + 16 * p) : u32x4_t{0u, 0u, 0u, 0u};
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) kv[16 * p + i] = (float)(int8_t)(ws[i / 4] >> (8 * (i % 4)));
      }
    } else {
      const int64_t base = (int64_t)h * a.k_stride_h + (int64_t)t * a.k_stride_t + c;
#pragma unroll
      for (int i = 0; i < 32; ++i)
        kv[i] = a.k_f32 ? reinterpret_cast<const float*>(a.k)[base + i]
                        : (float)reinterpret_cast<const _Float16*>(a.k)[base + i];
    }
#pragma unroll
    for (int i = 0; i < kMaxHeads; ++i) {
      const int g = wave + kWaves * i;
      if (g < G) {
        float s = acc[i];
#pragma unroll
        for (int d = 0; d < 32; ++d) s = fmaf(qs[g * D + c + d], kv[d], s);
        acc[i] = s;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxHeads; ++i) {
    const int g = wave + kWaves * i;
    if (g < G) a.logits[(int64_t)(h * G + g) * a.n + t] = acc[i] * kscale;
  }
}

// One workgroup per q head: the max of its logits, then the sum of
// exp(logit - max), each by a fixed-order tree over the 256 threads.
__global__ __launch_bounds__(256) void snapkv_stats_kernel(ScoreArgs a) {
  __shared__ float red[256];
  const int hq = blockIdx.x;
  const float* l = a.logits + (int64_t)hq * a.n;
  float m = -__builtin_inff();
  for (int t = threadIdx.x; t < a.n; t += 256) m = fmaxf(m, l[t]);
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  m = red[0];
  __syncthreads();
  float z = 0.0f;
  for (int t = threadIdx.x; t < a.n; t += 256) z += __expf(l[t] - m);
  red[threadIdx.x] = z;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    a.stats[2 * hq] = m;
    a.stats[2 * hq + 1] = red[0];
  }
}

__global__ __launch_bounds__(256) void snapkv_scores_kernel(ScoreArgs a) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.n) return;
  float s = 0.0f;
  for (int hq = 0; hq < a.num_q_heads; ++hq)
    s += __expf(a.logits[(int64_t)hq * a.n + t] - a.stats[2 * hq]) / a.stats[2 * hq + 1];
  a.scores[t] = s / (float)a.num_q_heads;
}

struct GatherArgs {
  char* base[8];
  int64_t row_words[8];     // 4-byte words per (token, head) row
  int64_t layer_stride[8];  // bytes between layers
  int num_layers, num_kv_heads, bs_log2;
  int64_t num_slots;        // num_blocks * block_size: valid flat slots are [0, num_slots)
  const int32_t* src;
  const int32_t* dst;
  int n;
};

__global__ __launch_bounds__(256) void gather_slots_kernel(GatherArgs a) {
  const int ti = blockIdx.z;
  const int layer = blockIdx.y;
  const int64_t W = a.row_words[ti];
  const int64_t total = (int64_t)a.n * a.num_kv_heads * W;
  uint32_t* p = reinterpret_cast<uint32_t*>(a.base[ti] + (int64_t)layer * a.layer_stride[ti]);
  const uint32_t bsm = (1u << a.bs_log2) - 1u;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t w = i % W;
    const int64_t r = i / W;
    const int h = (int)(r % a.num_kv_heads);
    const int64_t j = r / a.num_kv_heads;
    const int32_t s = a.src[j], d = a.dst[j];
    if (s < 0 || d < 0 || s >= a.num_slots || d >= a.num_slots) continue;  // outside the pool: nothing moves
    const int64_t sr = ((((int64_t)s >> a.bs_log2) * a.num_kv_heads + h) << a.bs_log2) + (s & bsm);
    const int64_t dr = ((((int64_t)d >> a.bs_log2) * a.num_kv_heads + h) << a.bs_log2) + (d & bsm);
    p[dr * W + w] = p[sr * W + w];
  }
}

template <int D, bool PAGED>
static int launch_scores(ScoreArgs& a, hipStream_t s) {
  const int lds = a.group * D * 4;
  if (lds > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&snapkv_logits_kernel<D, PAGED>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) {
      set_error("snapkv_scores: cannot raise the LDS limit");
      return S8KV_ERR_LAUNCH;
    }
  }
  hipLaunchKernelGGL((snapkv_logits_kernel<D, PAGED>), dim3((a.n + kTok - 1) / kTok, a.num_kv_heads),
                     dim3(64 * kWaves), lds, s, a);
  hipLaunchKernelGGL(snapkv_stats_kernel, dim3(a.num_q_heads), dim3(256), 0, s, a);
  hipLaunchKernelGGL(snapkv_scores_kernel, dim3((a.n + 255) / 256), dim3(256), 0, s, a);
  return check_launch("s8kv_snapkv_scores");
}

template <bool PAGED>
static int dispatch_scores(ScoreArgs& a, int head_dim, hipStream_t s) {
  switch (head_dim) {
    case 32: return launch_scores<32, PAGED>(a, s);
    case 64: return launch_scores<64, PAGED>(a, s);
    case 128: return launch_scores<128, PAGED>(a, s);
    case 256: return launch_scores<256, PAGED>(a, s);
  }
  set_error("snapkv_scores: head_dim %d not in {32,64,128,256}", head_dim);
  return S8KV_ERR_UNSUPPORTED;
}

static int score_common(ScoreArgs& a, int num_q_heads, int num_kv_heads, int head_dim, int n, void* workspace,
                        int64_t workspace_bytes, float* scores) {
  S8KV_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0, S8KV_ERR_INVALID,
               "snapkv_scores: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads, num_kv_heads);
  S8KV_REQUIRE(head_dim_ok(head_dim), S8KV_ERR_UNSUPPORTED, "snapkv_scores: head_dim %d not in {32,64,128,256}",
               head_dim);
  S8KV_REQUIRE(num_q_heads / num_kv_heads <= 4 * 16, S8KV_ERR_UNSUPPORTED,
               "snapkv_scores: more than 64 q heads per kv head");
  S8KV_REQUIRE((num_q_heads / num_kv_heads) * head_dim <= kMaxGroupDims, S8KV_ERR_UNSUPPORTED,
               "snapkv_scores: q heads per kv head x head_dim exceeds %d", kMaxGroupDims);
  S8KV_REQUIRE(n >= 0, S8KV_ERR_INVALID, "snapkv_scores: length < 0");
  const int64_t need = ((int64_t)num_q_heads * n + 2 * (int64_t)num_q_heads) * 4;
  S8KV_REQUIRE(workspace != nullptr && workspace_bytes >= need, S8KV_ERR_WORKSPACE,
               "snapkv_scores: workspace of %lld bytes needed, %lld given", (long long)need,
               (long long)workspace_bytes);
  S8KV_REQUIRE((uintptr_t)workspace % 4 == 0 && scores != nullptr, S8KV_ERR_INVALID,
               "snapkv_scores: null output or misaligned workspace");
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.n = n;
  a.logits = reinterpret_cast<float*>(workspace);
  a.stats = a.logits + (int64_t)num_q_heads * n;
  a.scores = scores;
  return S8KV_OK;
}

}  // namespace evict
}  // namespace s8kv

using namespace s8kv;

extern "C" int64_t s8kv_snapkv_workspace_size(int num_q_heads, int length) {
  if (num_q_heads <= 0 || length < 0) return 0;
  return ((int64_t)num_q_heads * length + 2 * (int64_t)num_q_heads) * 4;
}

extern "C" int s8kv_snapkv_scores_paged(const void* q, int q_is_f32, int64_t q_stride, int num_q_heads,
                                        int num_kv_heads, int head_dim, const int8_t* k_cache, const float* k_scale,
                                        int64_t num_blocks, int block_size, const int32_t* block_row, int length,
                                        float scale, float* scores, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
  evict::ScoreArgs a{};
  int rc = evict::score_common(a, num_q_heads, num_kv_heads, head_dim, length, workspace, workspace_bytes, scores);
  if (rc != S8KV_OK) return rc;
  if (length == 0) return S8KV_OK;
  S8KV_REQUIRE(q && k_cache && k_scale && block_row, S8KV_ERR_INVALID, "snapkv_scores_paged: null pointer argument");
  S8KV_REQUIRE(is_pow2(block_size) && block_size >= 4, S8KV_ERR_UNSUPPORTED,
               "snapkv_scores_paged: block_size %d must be a power of two >= 4", block_size);
  S8KV_REQUIRE(q_stride >= head_dim && num_blocks > 0, S8KV_ERR_INVALID, "snapkv_scores_paged: bad q stride or pool");
  S8KV_REQUIRE((uintptr_t)k_cache % 16 == 0, S8KV_ERR_INVALID, "snapkv_scores_paged: k_cache not 16-byte aligned");
  a.q = q;
  a.q_f32 = q_is_f32 ? 1 : 0;
  a.q_stride = q_stride;
  a.scale = scale;
  a.rot_norm = (float)(1.0 / __builtin_sqrt((double)head_dim));
  a.k_cache = k_cache;
  a.k_scale = k_scale;
  a.num_blocks = num_blocks;
  a.block_row = block_row;
  a.bs_log2 = log2i(block_size);
  return evict::dispatch_scores<true>(a, head_dim, (hipStream_t)stream);
}

extern "C" int s8kv_snapkv_scores_dense(const void* q, int q_is_f32, int64_t q_stride, int num_q_heads,
                                        int num_kv_heads, int head_dim, const void* k, int k_is_f32,
                                        int64_t k_stride_h, int64_t k_stride_t, int length, float scale, float* scores,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  evict::ScoreArgs a{};
  int rc = evict::score_common(a, num_q_heads, num_kv_heads, head_dim, length, workspace, workspace_bytes, scores);
  if (rc != S8KV_OK) return rc;
  if (length == 0) return S8KV_OK;
  S8KV_REQUIRE(q && k, S8KV_ERR_INVALID, "snapkv_scores_dense: null pointer argument");
  S8KV_REQUIRE(q_stride >= head_dim && k_stride_t >= head_dim, S8KV_ERR_INVALID,
               "snapkv_scores_dense: row strides must be >= head_dim");
  a.q = q;
  a.q_f32 = q_is_f32 ? 1 : 0;
  a.q_stride = q_stride;
  a.scale = scale;
  a.k = k;
  a.k_f32 = k_is_f32 ? 1 : 0;
  a.k_stride_h = k_stride_h;
  a.k_stride_t = k_stride_t;
  return evict::dispatch_scores<false>(a, head_dim, (hipStream_t)stream);
}

extern "C" int s8kv_gather_slots(int num_tensors, void* const* tensor_ptrs, const int64_t* row_bytes,
                                 const int64_t* layer_stride_bytes, int num_layers, int num_kv_heads,
                                 int64_t num_blocks, int block_size, const int32_t* src_slots,
                                 const int32_t* dst_slots, int num_tokens, void* stream) {
  S8KV_REQUIRE(num_tensors >= 1 && num_tensors <= 8, S8KV_ERR_INVALID, "gather_slots: 1..8 tensors, got %d",
               num_tensors);
  S8KV_REQUIRE(num_layers >= 1 && num_kv_heads >= 1 && num_blocks >= 1 && num_tokens >= 0, S8KV_ERR_INVALID,
               "gather_slots: bad geometry");
  S8KV_REQUIRE(is_pow2(block_size) && block_size >= 1, S8KV_ERR_UNSUPPORTED,
               "gather_slots: block_size %d must be a power of two", block_size);
  if (num_tokens == 0) return S8KV_OK;
  S8KV_REQUIRE(tensor_ptrs && row_bytes && layer_stride_bytes && src_slots && dst_slots, S8KV_ERR_INVALID,
               "gather_slots: null pointer argument");
  evict::GatherArgs a{};
  int64_t max_words = 0;
  for (int i = 0; i < num_tensors; ++i) {
    S8KV_REQUIRE(tensor_ptrs[i] != nullptr && (uintptr_t)tensor_ptrs[i] % 4 == 0, S8KV_ERR_INVALID,
                 "gather_slots: tensor %d null or not 4-byte aligned", i);
    S8KV_REQUIRE(row_bytes[i] > 0 && row_bytes[i] % 4 == 0 && layer_stride_bytes[i] % 4 == 0, S8KV_ERR_INVALID,
                 "gather_slots: tensor %d row bytes / layer stride not multiples of 4", i);
    S8KV_REQUIRE(layer_stride_bytes[i] >= num_blocks * num_kv_heads * block_size * row_bytes[i] || num_layers == 1,
                 S8KV_ERR_INVALID, "gather_slots: tensor %d layer stride smaller than a layer", i);
    a.base[i] = static_cast<char*>(tensor_ptrs[i]);
    a.row_words[i] = row_bytes[i] / 4;
    a.layer_stride[i] = layer_stride_bytes[i];
    if (a.row_words[i] > max_words) max_words = a.row_words[i];
  }
  a.num_layers = num_layers;
  a.num_kv_heads = num_kv_heads;
  a.bs_log2 = log2i(block_size);
  a.num_slots = num_blocks * block_size;
  a.src = src_slots;
  a.dst = dst_slots;
  a.n = num_tokens;
  const int64_t work = (int64_t)num_tokens * num_kv_heads * max_words;
  const int64_t blocks = (work + 255) / 256 < 4096 ? (work + 255) / 256 : 4096;
  S8KV_REQUIRE(num_layers <= 65535, S8KV_ERR_UNSUPPORTED, "gather_slots: more than 65535 layers");
  hipLaunchKernelGGL(evict::gather_slots_kernel, dim3((unsigned)blocks, num_layers, num_tensors), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("s8kv_gather_slots");
}
