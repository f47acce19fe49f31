// Whole-block copy across every layer of the cache tensors (copy-on-write of a
// shared prefix block, pool compaction).  Pure HBM streaming: each workgroup
// moves one 8 KiB chunk of one (tensor, block pair, layer); every thread
// issues its two 16-byte loads (4 KiB apart, so each instruction is one
// contiguous 4 KiB span per workgroup) before its two non-temporal stores.
// Two loads in flight per thread measured fastest (1, 4 and 8 are slower).
#include "s8kv_device.h"
#include "s8kv_host.h"

namespace s8kv {

constexpr int kMaxCopyTensors = 8;
constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 2;
constexpr int kCopyStep = kCopyThreads * 16;            // bytes per load instruction of the workgroup
constexpr int kCopyChunk = kCopyStep * kCopyUnroll;     // bytes per workgroup

struct CopyArgs {
  char* base[kMaxCopyTensors];
  int64_t block_bytes[kMaxCopyTensors];
  int64_t layer_stride[kMaxCopyTensors];
  int chunk_begin[kMaxCopyTensors + 1];  // prefix sum of chunks per tensor
  int vec16[kMaxCopyTensors];            // base, layer stride and block bytes all 16-byte aligned
  int num_tensors;
  int64_t num_blocks;
  const int32_t* src;
  const int32_t* dst;
};

__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(CopyArgs a) {
  const int chunk_id = blockIdx.x;
  const int pair = blockIdx.y;
  const int layer = blockIdx.z;
  int t = 0;
  while (t + 1 < a.num_tensors && chunk_id >= a.chunk_begin[t + 1]) ++t;
  const int32_t sb = a.src[pair];
  const int32_t db = a.dst[pair];
  if (sb < 0 || db < 0 || sb >= a.num_blocks || db >= a.num_blocks) return;
  const int64_t bb = a.block_bytes[t];
  const int64_t off0 = (int64_t)(chunk_id - a.chunk_begin[t]) * kCopyChunk + (int64_t)threadIdx.x * 16;
  if (off0 >= bb) return;
  const char* s = a.base[t] + layer * a.layer_stride[t] + (int64_t)sb * bb;
  char* d = a.base[t] + layer * a.layer_stride[t] + (int64_t)db * bb;
  if (a.vec16[t]) {  // 16-byte aligned blocks: vector moves, all loads in flight first
    u32x4_t v[kCopyUnroll];
#pragma unroll
    for (int i = 0; i < kCopyUnroll; ++i) {
      const int64_t off = off0 + (int64_t)i * kCopyStep;
      if (off < bb) v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(s + off));
    }
#pragma unroll
    for (int i = 0; i < kCopyUnroll; ++i) {
      const int64_t off = off0 + (int64_t)i * kCopyStep;
      if (off < bb) __builtin_nontemporal_store(v[i], reinterpret_cast<u32x4_t*>(d + off));
    }
  } else {
    for (int i = 0; i < kCopyUnroll; ++i) {
      const int64_t off = off0 + (int64_t)i * kCopyStep;
      for (int64_t k = 0; k < 16 && off + k + 4 <= bb; k += 4)
        *reinterpret_cast<uint32_t*>(d + off + k) = *reinterpret_cast<const uint32_t*>(s + off + k);
    }
  }
}

}  // namespace s8kv

using namespace s8kv;

extern "C" int s8kv_copy_blocks(int num_tensors, void* const* tensor_ptrs, const int64_t* block_bytes,
                                const int64_t* layer_stride_bytes, int num_layers, int64_t num_blocks,
                                const int32_t* src_blocks, const int32_t* dst_blocks, int num_pairs, void* stream) {
  S8KV_REQUIRE(num_tensors > 0 && num_tensors <= kMaxCopyTensors, S8KV_ERR_INVALID,
               "copy_blocks: num_tensors %d not in [1, %d]", num_tensors, kMaxCopyTensors);
  S8KV_REQUIRE(num_pairs >= 0 && num_layers >= 0, S8KV_ERR_INVALID, "copy_blocks: negative count");
  if (num_pairs == 0 || num_layers == 0) return S8KV_OK;
  S8KV_REQUIRE(tensor_ptrs && block_bytes && layer_stride_bytes && src_blocks && dst_blocks, S8KV_ERR_INVALID,
               "copy_blocks: null pointer argument");
  S8KV_REQUIRE(num_layers <= 65535 && num_pairs <= 65535, S8KV_ERR_UNSUPPORTED,
               "copy_blocks: at most 65535 layers and block pairs per call");
  CopyArgs a{};
  a.num_tensors = num_tensors;
  a.num_blocks = num_blocks;
  a.src = src_blocks;
  a.dst = dst_blocks;
  int chunks = 0;
  for (int i = 0; i < num_tensors; ++i) {
    S8KV_REQUIRE(tensor_ptrs[i] != nullptr, S8KV_ERR_INVALID, "copy_blocks: tensor %d is null", i);
    S8KV_REQUIRE(block_bytes[i] > 0 && block_bytes[i] % 4 == 0, S8KV_ERR_INVALID,
                 "copy_blocks: block_bytes[%d]=%lld must be a positive multiple of 4", i, (long long)block_bytes[i]);
    S8KV_REQUIRE(layer_stride_bytes[i] >= block_bytes[i] * num_blocks, S8KV_ERR_INVALID,
                 "copy_blocks: layer stride of tensor %d smaller than num_blocks * block_bytes", i);
    a.base[i] = (char*)tensor_ptrs[i];
    a.block_bytes[i] = block_bytes[i];
    a.layer_stride[i] = layer_stride_bytes[i];
    a.vec16[i] = ((reinterpret_cast<uintptr_t>(tensor_ptrs[i]) | (uintptr_t)layer_stride_bytes[i] |
                   (uintptr_t)block_bytes[i]) & 15) == 0;
    a.chunk_begin[i] = chunks;
    chunks += (int)((block_bytes[i] + kCopyChunk - 1) / kCopyChunk);
  }
  a.chunk_begin[num_tensors] = chunks;
  dim3 grid(chunks, num_pairs, num_layers);
  hipLaunchKernelGGL(copy_blocks_kernel, grid, dim3(kCopyThreads), 0, (hipStream_t)stream, a);
  return check_launch("s8kv_copy_blocks");
}
