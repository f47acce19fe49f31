// Diagnostics (no counterpart in the reference): read-only HBM streaming
// probes that bound what a kernel reading the same bytes can reach.
//
// s8kv_probe_read_tiles reads exactly the bytes a decode launch reads from the
// paged cache -- for every listed 32-token tile of a (row, KV head), its K
// and V rows and their scales -- with the decode kernel's shape: about as
// many 4-wave workgroups as stay resident, each taking an equal contiguous
// share of the tile list, waves taking tiles in turn with the next tile's
// loads in flight while the current one is folded into a checksum; the loads
// are non-temporal, as the decode kernel's.
// s8kv_probe_read_linear reads one contiguous buffer the same way (16-byte
// loads, four in flight per lane).  Each workgroup writes one checksum word,
// so no load can be dropped.
#include "s8kv_device.h"
#include "s8kv_host.h"

namespace s8kv {
namespace diag {

constexpr int kWaves = 4;

struct TileProbeArgs {
  const void* k_cache;
  const void* v_cache;
  const void* k_scale;
  const void* v_scale;
  uint32_t kc_bytes, ks_bytes;
  const int32_t* tiles;   // first storage row of each tile (32 rows, one block, one head)
  int ntiles;
  int head_dim;           // 128
  int nwg;
  uint32_t* sink;
};

struct TileRegs {
  u32x4_t k[4], v[4];
  uint32_t ks, vs;
};

__device__ __forceinline__ void load_tile(const TileProbeArgs& a, rsrc_t kc, rsrc_t vc, rsrc_t ks, rsrc_t vs,
                                          int t, int lane, TileRegs& r) {
  const uint32_t row0 = (uint32_t)a.tiles[t];
  // 32 rows x 128 B = 4 KiB per tensor: 4 loads of 64 lanes x 16 B
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t off = row0 * 128u + (uint32_t)(i * 1024 + lane * 16);
    r.k[i] = bload128<kNT>(kc, off);
    r.v[i] = bload128<kNT>(vc, off);
  }
  r.ks = bload32<kNT>(ks, row0 * 4u + (uint32_t)(lane & 31) * 4u);
  r.vs = bload32<kNT>(vs, row0 * 4u + (uint32_t)(lane & 31) * 4u);
}

__device__ __forceinline__ uint32_t fold(const TileRegs& r) {
  uint32_t x = r.ks ^ r.vs;
#pragma unroll
  for (int i = 0; i < 4; ++i) x ^= r.k[i].x ^ r.k[i].y ^ r.k[i].z ^ r.k[i].w ^ r.v[i].x ^ r.v[i].y ^ r.v[i].z ^ r.v[i].w;
  return x;
}

__global__ __launch_bounds__(64 * kWaves) void probe_tiles_kernel(TileProbeArgs a) {
  const int j = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t0 = (int)((int64_t)a.ntiles * j / a.nwg);
  const int t1 = (int)((int64_t)a.ntiles * (j + 1) / a.nwg);
  const rsrc_t kc = make_rsrc(a.k_cache, a.kc_bytes);
  const rsrc_t vc = make_rsrc(a.v_cache, a.kc_bytes);
  const rsrc_t ks = make_rsrc(a.k_scale, a.ks_bytes);
  const rsrc_t vs = make_rsrc(a.v_scale, a.ks_bytes);
  uint32_t acc = 0;
  int t = t0 + wave;
  if (t < t1) {
    TileRegs cur, nxt;
    load_tile(a, kc, vc, ks, vs, t, lane, cur);
    for (; t + kWaves < t1; t += kWaves) {
      load_tile(a, kc, vc, ks, vs, t + kWaves, lane, nxt);
      acc ^= fold(cur);
      cur = nxt;
    }
    acc ^= fold(cur);
  }
  __shared__ uint32_t red[64 * kWaves];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
    for (int i = 0; i < 64 * kWaves; ++i) x ^= red[i];
    a.sink[j] = x;
  }
}

__global__ __launch_bounds__(64 * kWaves) void probe_linear_kernel(const u32x4_t* p, int64_t n16, int nwg,
                                                                   uint32_t* sink) {
  const int j = blockIdx.x;
  const int64_t lo = n16 * j / nwg, hi = n16 * (j + 1) / nwg;
  uint32_t acc = 0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += 4 * 64 * kWaves) {
    u32x4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t k = i + (int64_t)u * 64 * kWaves;
      v[u] = k < hi ? __builtin_nontemporal_load(p + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  __shared__ uint32_t red[64 * kWaves];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
    for (int i = 0; i < 64 * kWaves; ++i) x ^= red[i];
    sink[j] = x;
  }
}

}  // namespace diag
}  // namespace s8kv

using namespace s8kv;

extern "C" int s8kv_probe_read_tiles(const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                                     const float* v_scale, int64_t num_rows, int head_dim, const int32_t* tiles,
                                     int num_tiles, int num_workgroups, uint32_t* sink, void* stream) {
  S8KV_REQUIRE(head_dim == 128, S8KV_ERR_UNSUPPORTED, "probe_read_tiles: head_dim %d != 128", head_dim);
  S8KV_REQUIRE(k_cache && k_scale && v_cache && v_scale && tiles && sink, S8KV_ERR_INVALID,
               "probe_read_tiles: null pointer argument");
  S8KV_REQUIRE(num_tiles >= 0 && num_workgroups >= 1 && num_workgroups <= 65535 * 8, S8KV_ERR_INVALID,
               "probe_read_tiles: bad sizes");
  S8KV_REQUIRE(fits_u32(num_rows * head_dim), S8KV_ERR_UNSUPPORTED, "probe_read_tiles: cache exceeds 4 GiB");
  diag::TileProbeArgs a{};
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.kc_bytes = (uint32_t)(num_rows * head_dim);
  a.ks_bytes = (uint32_t)(num_rows * 4);
  a.tiles = tiles;
  a.ntiles = num_tiles;
  a.head_dim = head_dim;
  a.nwg = num_workgroups;
  a.sink = sink;
  hipLaunchKernelGGL(diag::probe_tiles_kernel, dim3(num_workgroups), dim3(64 * diag::kWaves), 0, (hipStream_t)stream,
                     a);
  return check_launch("s8kv_probe_read_tiles");
}

extern "C" int s8kv_probe_read_linear(const void* buffer, int64_t bytes, int num_workgroups, uint32_t* sink,
                                      void* stream) {
  S8KV_REQUIRE(buffer && sink && bytes >= 0 && bytes % 16 == 0 && (uintptr_t)buffer % 16 == 0, S8KV_ERR_INVALID,
               "probe_read_linear: buffer must be 16-byte aligned, its size a multiple of 16");
  S8KV_REQUIRE(num_workgroups >= 1 && num_workgroups <= 65535 * 8, S8KV_ERR_INVALID, "probe_read_linear: bad grid");
  hipLaunchKernelGGL(diag::probe_linear_kernel, dim3(num_workgroups), dim3(64 * diag::kWaves), 0,
                     (hipStream_t)stream, static_cast<const u32x4_t*>(buffer), bytes / 16, num_workgroups, sink);
  return check_launch("s8kv_probe_read_linear");
}
