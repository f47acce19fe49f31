// Multi-query verify attention over the paged int8 or K8V3 cache: tree verify (each
// draft query sees the prefix plus its ancestors in the draft tree) and
// chunked prefill / chain verify (query s sees the prefix plus drafts 0..s).
//
// Layout of the work: a workgroup of W waves (4; 8 for K8V3) owns 16 * W * RG
// query rows of one (sequence, KV head) pair -- row r is query position r / G of q head
// h*G + r % G -- and streams the pair's keys in 32-key tiles.  Each tile's K
// and V rows are loaded once per workgroup, converted int8 -> fp16 (exact) on
// the way into LDS (double-buffered), and shared by its waves (K8V3: V's
// 3-bit codes become the fp16 codebook entries, as in the decode kernel); a
// wave owns RG groups of 16 query rows (RG = 2 for head_dim 64, else 1),
// each group the 16 columns of its own MFMA tiles, and every K and V operand a
// wave reads from LDS feeds the MFMAs of all its groups:
//   QK  : S^T[key][row] on MFMA 16x16x32 f16, A = K rows from LDS, B = the
//         rotated, pre-scaled q split into fp16 hi + lo (two MFMAs); dense
//         inputs: the fp16 q itself (one MFMA), the scale applied to the score.
//   mask: keys below the prefix are visible to every row; draft key i is
//         visible to row position s if i <= s (chain) or bit i of the row's
//         tree mask is set (tree).
//   softmax: online, log2 domain, lazy max (as the decode kernel): a score
//         enters as y = s * k_scale - m in one FMA; a tile whose y exceeds
//         the slack recomputes the running max from the products.
//   PV  : O^T[dim][row] on MFMA, A = V^T via ds_read_b64_tr_b16 from LDS,
//         B = P * v_scale (K8V3: P * the key's block norm) as fp16 hi + lo
//         (hi: the fp32 weight cut to fp16 precision, lo: the exact rest).
// Rows past a sequence's query count are written as zeros.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "s8kv_device.h"
#include "s8kv_host.h"

namespace s8kv {
namespace verify {

// Waves per workgroup: 4, or 8 for the K8V3 layout, whose V-code expansion
// into LDS (VALU work per tile) is then shared by twice the query rows.
template <bool K8V3> constexpr int kWavesOf = K8V3 ? 8 : 4;
constexpr int kTile = 32;
constexpr int kSubKeys = 2048;                 // block ids staged in LDS per 2048 keys
constexpr int kMaxSubBlocks = kSubKeys / 4 + 2;  // block_size >= 4
constexpr float kNegInf = -__builtin_inff();
constexpr float kMaxSlack = 8.0f;
// Running max before any key: finite, so exp2(score - max) is 0 for a masked
// score (-inf) and never NaN, with no test per score; any real score exceeds
// it by more than kMaxSlack + esh, which makes the first visible tile rescale (by 0).
constexpr float kMaxInit = -1.0e30f;

template <int D, bool K8V3>
struct Cfg {
  static constexpr int RG = D <= 64 ? 2 : 1;         // 16-row groups per wave (as registers allow)
  static constexpr int WAVES = kWavesOf<K8V3>;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS = 16 * RG * WAVES;       // query rows per workgroup
  static constexpr int KCH = D / 4;      // dims per lane per key row (MFMA A / B chunk of the lane group)
  static constexpr int NQK = D / 32;     // QK MFMAs per 16-key subtile
  static constexpr int NPV = D / 16;     // PV MFMAs per tile
  static constexpr int KROW = 2 * D + 16;  // LDS pitch of an fp16 K row (bytes)
  static constexpr int VROW = 2 * D + 32;  // LDS pitch of an fp16 V row (bytes)
  static constexpr int KBYTES = kTile * KROW;
  static constexpr int VBYTES = kTile * VROW;
  static constexpr int NB = K8V3 ? D / 128 : 1;  // V scales per key: the int8 row scale, or K8V3 block norms
  static constexpr int NG = D / 32;              // K8V3: 32-value code groups per key (3 packed words each)
  static constexpr int WORDS = 3 * NG;           // K8V3: packed words per key
  static constexpr int SBYTES = (1 + NB) * kTile * 4;  // k_scale, then the V scales of each block
  static constexpr int BUF = KBYTES + VBYTES + SBYTES;
  static constexpr int CHUNKS = kTile * D / 16;                 // 16-byte int8 chunks per K (or V) tile
  static constexpr int LOADS = (CHUNKS + THREADS - 1) / THREADS;
  static constexpr int CHUNKS_F16 = kTile * D / 8;              // dense fp16 inputs: 16-byte chunks per tile
  static constexpr int LOADS_F16 = (CHUNKS_F16 + THREADS - 1) / THREADS;
  // K8V3: a code group's 32 values are expanded by SPLIT threads (16 values
  // each when the tile has fewer groups than the workgroup has threads)
  static constexpr int SPLIT = kTile * NG < THREADS ? (THREADS >= 2 * kTile * NG ? 2 : 1) : 1;
  static constexpr int VJOBS = kTile * NG * SPLIT;              // K8V3: expansion jobs per tile
  static_assert(!K8V3 || (VJOBS <= THREADS && (SPLIT == 1 || SPLIT == 2)), "one K8V3 job per thread");
  static constexpr int SMEM = 2 * BUF + kMaxSubBlocks * 4;
  // window verify with fresh drafts: the low fp16 part of the draft keys'
  // fp32 K, one K-sized tile per buffer after the block ids
  static constexpr int KLO_OFF = (SMEM + 15) / 16 * 16;
  static constexpr int SMEM_WIN = KLO_OFF + 2 * KBYTES;
};

struct VerifyArgs {
  const _Float16* q;
  int64_t q_stride_b, q_stride_h, q_stride_s;
  int batch, num_q_heads, num_kv_heads, group, max_queries;
  const void* k_cache;
  const float* k_scale;
  const void* v_cache;        // int8 V, or K8V3 packed code words
  const float* v_scale;       // int8 V scales, or K8V3 block norms
  const float* v_codebook;    // K8V3: fp32 [8]
  uint32_t kc_bytes, ks_bytes, vc_bytes, vs_bytes;
  // the tensors' full sizes; verify_kernel<.., BIG> (a tensor past 4 GiB,
  // block_size >= 32) loads each tile through descriptors rebased to it
  uint64_t kc_total, ks_total, vc_total, vs_total;
  int big;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* prefix_lens;
  const int32_t* query_lens;  // nullable: every row has max_queries queries
  const int64_t* tree_mask;   // nullable: chain; else [batch][max_queries] ancestor bits
  int bs_log2;
  int max_context_len;
  int n_qblocks;              // query blocks (rows_per_wg rows each) per (sequence, KV head)
  // split of the key range: workgroup split sp of a (sequence, KV head, query
  // block) attends its share of the keys and writes unnormalized partials
  // (acc[D], m_ref, l per row, pitch D + 4 floats) to part; a second kernel
  // combines them.  splits == 1: the workgroup writes the output itself.
  int splits;
  float* part;
  int window;                 // verify_kernel<.., WIN>: only the last `window` prefix keys are visible
  // WIN, optional: the drafts' fresh K (rotated, fp32) and V (fp16),
  // attended in place of their cache rows (draft i of row b, head h at
  // b * stride_b + i * stride_s + h * stride_h; head_dim contiguous)
  const float* kd;
  const _Float16* vd;
  int64_t kd_stride_b, kd_stride_s, kd_stride_h, vd_stride_b, vd_stride_s, vd_stride_h;
  // dense inputs (verify_kernel<D, false, false, true>: prefill attention over
  // fresh fp16 K / V, token-major, sequences delimited by cu_seqlens)
  const int32_t* cu_q;
  const int32_t* cu_k;
  const _Float16* k_f16;
  const _Float16* v_f16;
  int64_t k_stride_t, k_stride_h, v_stride_t, v_stride_h, o_stride_t, o_stride_h;
  int causal;
  float qscale;
  _Float16* out;              // [batch][Hq][max_queries][D]
};

// Position of tile key tt (0..31) in the LDS V tile: lane group g's eight
// transpose-read rows (keys 4g..4g+3 and 16+4g..16+4g+3) are rows 8g..8g+7.
__device__ __forceinline__ int vrow_of(int tt) { return 8 * ((tt & 15) >> 2) + 4 * (tt >> 4) + (tt & 3); }

template <int D, bool K8V3, bool WIN = false, bool DENSE = false, bool BIG = false>
__global__ __launch_bounds__(64 * kWavesOf<K8V3>, K8V3 ? 1 : 2) void verify_kernel(VerifyArgs a) {
  static_assert(!DENSE || !K8V3, "dense inputs: fp16 K / V");
  static_assert(!DENSE || !BIG, "dense inputs are not paged");
  using C = Cfg<D, K8V3>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int* bt_lds = reinterpret_cast<int*>(smem + 2 * C::BUF);

  // workgroups of one (sequence, KV head) pair share an XCD (and its L2)
  const int P = a.batch * a.num_kv_heads;
  const int xcd = blockIdx.x & 7;
  const int rest = blockIdx.x >> 3;
  const int qb = rest % a.n_qblocks;
  const int rest2 = rest / a.n_qblocks;
  const int sp = rest2 % a.splits;
  const int p = (rest2 / a.splits) * 8 + xcd;
  if (p >= P) return;
  const int b = p / a.num_kv_heads;
  const int h = p - b * a.num_kv_heads;
  const int G = a.group;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  // dense: sequence b's queries are tokens cu_q[b] .., its keys cu_k[b] ..;
  // causal is bottom-right aligned (query s sees keys j <= s + nk - nq, which
  // may be none), else every key is visible.  The diagonal comes from the
  // sequence's own counts; max_queries (max_seqlen_q) only sizes the grid, so
  // queries past it are not computed (the entry point requires it to bound
  // every sequence), and max_seqlen_k is not used to clamp the keys.
  int nq, prefix, nk = 0, q0 = 0, k0 = 0;
  if constexpr (DENSE) {
    q0 = a.cu_q[b];
    k0 = a.cu_k[b];
    const int nq_seq = max(0, a.cu_q[b + 1] - q0);
    nk = max(0, a.cu_k[b + 1] - k0);
    nq = min(nq_seq, a.max_queries);
    prefix = a.causal ? nk - nq_seq : nk;
  } else {
    nq = a.query_lens ? max(0, min(a.query_lens[b], a.max_queries)) : a.max_queries;
    prefix = max(0, a.prefix_lens[b]);
  }
  constexpr int RG = C::RG;
  const int row0 = qb * C::ROWS;                    // first row of the workgroup
  const int pos_hi = min(nq, (row0 + C::ROWS + G - 1) / G);  // positions of this block that exist
  const bool tree = a.tree_mask != nullptr;
  // keys any row of this block can see
  int kv_end = prefix + (tree ? nq : pos_hi);
  kv_end = min(kv_end, DENSE ? nk : a.max_context_len);
  if (row0 / G >= nq) kv_end = 0;  // no query of this block exists
  // sliding window: prefix keys below lo_key are invisible to every row; the
  // key loop starts at the 32-key tile holding lo_key, whose lower keys are masked
  // (dense inputs: a band -- query s sees keys j >= prefix + s - window, so the
  // block's loop starts at its first position's bound and keys from its last
  // position's bound on are visible to every row)
  const int lo_key = WIN ? max(0, prefix + (DENSE ? row0 / G : 0) - a.window) : 0;
  const int lo_all = WIN && DENSE ? prefix + min(nq - 1, (row0 + C::ROWS - 1) / G) - a.window : lo_key;
  // keys below vis_all are visible to every row of the block: the prefix, and
  // for a chain / causal block also the drafts up to its first position
  const int vis_all = tree ? prefix : prefix + row0 / G + 1;

  // this lane's column in each of its row groups: query row r -> (position, q head)
  int pos[RG], head[RG];
  bool row_live[RG];
  uint64_t tmask[RG];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const int r = row0 + (rg * C::WAVES + wave) * 16 + c;
    pos[rg] = r / G;
    head[rg] = h * G + (r - pos[rg] * G);
    row_live[rg] = pos[rg] < nq;
    tmask[rg] = (tree && row_live[rg]) ? (uint64_t)a.tree_mask[(int64_t)b * a.max_queries + pos[rg]] : 0ull;
  }

  // ---- q: rotate (FWHT), pre-scale, split into fp16 hi + lo ----
  half8_t qhi[RG][C::NQK], qlo[RG][C::NQK];
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    float x[C::KCH];
    const int64_t qrow = DENSE ? (int64_t)q0 * a.q_stride_s : (int64_t)b * a.q_stride_b;
    const _Float16* qp = a.q + qrow + (int64_t)head[rg] * a.q_stride_h +
                         (int64_t)(row_live[rg] ? pos[rg] : 0) * a.q_stride_s + g * C::KCH;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) x[i] = row_live[rg] ? (float)qp[i] : 0.0f;
    // dense inputs: K is not rotated, so neither is q
#pragma unroll
    for (int hs = 1; hs < (DENSE ? 1 : C::KCH); hs <<= 1) {
#pragma unroll
      for (int i = 0; i < C::KCH; ++i) {
        if ((i & hs) == 0) {
          const float x0 = x[i], x1 = x[i + hs];
          x[i] = x0 + x1;
          x[i + hs] = x0 - x1;
        }
      }
    }
    if constexpr (!DENSE) {
#pragma unroll
      for (int i = 0; i < C::KCH; ++i) x[i] = butterfly_x16(x[i], lane);
#pragma unroll
      for (int i = 0; i < C::KCH; ++i) x[i] = butterfly_x32(x[i], lane);
    }
#pragma unroll
    for (int m = 0; m < C::NQK; ++m) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // (materialized: hi and lo must both come from this one fp32 value; a
        // fused fp16(x*s) for the lo term can differ from fp16(val) by one ulp)
        if constexpr (DENSE) {  // q is the fp16 input: exact; the scale multiplies the fp32 score
          qhi[rg][m][e] = (_Float16)x[8 * m + e];
          qlo[rg][m][e] = (_Float16)0.0f;
          continue;
        }
        const float val = materialize(x[8 * m + e] * a.qscale);
        const _Float16 qh = (_Float16)val;
        qhi[rg][m][e] = qh;
        qlo[rg][m][e] = (_Float16)(val - (float)qh);
      }
    }
  }

  float m_ref[RG], l_run[RG];  // m_ref: running max - esh (WeightShift)
  float4_t acc[RG][C::NPV];
  WeightShift ws(kMaxSlack);
  if constexpr (DENSE) ws.raise(1.0f, kMaxSlack);  // fp16 K / V: every V scale is 1
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    m_ref[rg] = kMaxInit;
    l_run[rg] = 0.0f;
#pragma unroll
    for (int n = 0; n < C::NPV; ++n) acc[rg][n] = float4_t{0.f, 0.f, 0.f, 0.f};
  }

  const rsrc_t kc = make_rsrc(a.k_cache, a.kc_bytes);
  const rsrc_t vc = make_rsrc(a.v_cache, a.vc_bytes);
  const rsrc_t ks = make_rsrc(a.k_scale, a.ks_bytes);
  const rsrc_t vs = make_rsrc(a.v_scale, a.vs_bytes);
  // K8V3 codebook byte tables (fp16 of the fp32 codebook; the decode kernel's)
  uint32_t tlo03 = 0, tlo47 = 0, thi03 = 0, thi47 = 0;
  if constexpr (K8V3) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t hb = __builtin_bit_cast(uint16_t, (_Float16)a.v_codebook[i]);
      const uint32_t lw = hb & 0xFFu, hw = hb >> 8;
      if (i < 4) { tlo03 |= lw << (8 * i); thi03 |= hw << (8 * i); }
      else { tlo47 |= lw << (8 * (i - 4)); thi47 |= hw << (8 * (i - 4)); }
    }
  }
  const int bs_log2 = a.bs_log2;
  const uint32_t bsm = (1u << bs_log2) - 1u;
  const uint32_t hkv = (uint32_t)a.num_kv_heads;
  const int32_t* bt_row = a.block_table + (int64_t)b * a.bt_stride;

  // this workgroup's keys: split sp of the block's tile-aligned key range
  int k_lo = lo_key & ~(kTile - 1), k_hi = kv_end;
  if (a.splits > 1) {
    const int chunk = ((max(0, kv_end - k_lo) + a.splits - 1) / a.splits + kTile - 1) & ~(kTile - 1);
    k_lo += sp * chunk;
    k_hi = min(kv_end, k_lo + chunk);
  }
  for (int u0 = k_lo; u0 < k_hi; u0 += kSubKeys) {
    const int u1 = min(k_hi, u0 + kSubKeys);
    const int fb = u0 >> bs_log2;
    const int nblk = ((u1 - 1) >> bs_log2) - fb + 1;
    __syncthreads();  // previous users of bt_lds and the tile buffers are done
    if constexpr (!DENSE)
      for (int i = tid; i < nblk; i += C::THREADS) bt_lds[i] = bt_row[fb + i];
    __syncthreads();

    // storage row of key kk (clamped to the last key, so every address is a real row)
    auto row_of = [&](int kk) -> uint32_t {
      kk = min(kk, u1 - 1);
      const uint32_t blk = (uint32_t)bt_lds[(kk >> bs_log2) - fb];
      return ((blk * hkv + (uint32_t)h) << bs_log2) + ((uint32_t)kk & bsm);
    };

    // ---- cooperative tile load: int8 K/V chunks (K8V3: a code group's three
    // words per thread) and scales -> registers ----
    constexpr int NREG = DENSE ? C::LOADS_F16 : C::LOADS;
    struct TileRegs {
      u32x4_t k[NREG], v[NREG];
      float s;
    };
    auto load_tile = [&](TileRegs& R, int base) {
      if constexpr (DENSE) {  // fp16 K / V rows of keys base .. base+31 (clamped to the last key)
#pragma unroll
        for (int i = 0; i < C::LOADS_F16; ++i) {
          const int ch = tid + i * C::THREADS;
          if (ch < C::CHUNKS_F16) {
            const int tt = ch / (D / 8), part = ch % (D / 8);
            const int64_t tok = k0 + min(base + tt, nk - 1);
            R.k[i] = *reinterpret_cast<const u32x4_t*>(a.k_f16 + tok * a.k_stride_t + h * a.k_stride_h + part * 8);
            R.v[i] = *reinterpret_cast<const u32x4_t*>(a.v_f16 + tok * a.v_stride_t + h * a.v_stride_h + part * 8);
          }
        }
        R.s = 1.0f;
        return;
      }
      if constexpr (BIG) {  // one block holds the tile (block_size >= 32): descriptors rebased to its first row
        const uint32_t r0 = __builtin_amdgcn_readfirstlane(row_of(base));
        auto local = [&](int tt) -> uint32_t { return (uint32_t)(min(base + tt, u1 - 1) - base); };
        const rsrc_t kt = window_rsrc(a.k_cache, a.kc_total, (uint64_t)r0 * D);
        const rsrc_t vt = window_rsrc(a.v_cache, a.vc_total, (uint64_t)r0 * (K8V3 ? C::WORDS * 4 : D));
        const rsrc_t kst = window_rsrc(a.k_scale, a.ks_total, (uint64_t)r0 * 4u);
        const rsrc_t vst = window_rsrc(a.v_scale, a.vs_total, (uint64_t)r0 * (C::NB * 4u));
#pragma unroll
        for (int i = 0; i < C::LOADS; ++i) {
          const int ch = tid + i * C::THREADS;
          if (ch < C::CHUNKS) {
            const int tt = ch / (D / 16), part = ch % (D / 16);
            const uint32_t off = local(tt) * (uint32_t)D + (uint32_t)part * 16u;
            R.k[i] = bload128(kt, off);
            if constexpr (!K8V3) R.v[i] = bload128(vt, off);
          }
        }
        if constexpr (K8V3) {
          if (tid < C::VJOBS) {
            const int grp = tid / C::SPLIT;
            const int tt = grp / C::NG, gi = grp % C::NG;
            const uint32_t off = local(tt) * (uint32_t)(C::WORDS * 4) + (uint32_t)gi * 12u;
            const u32x3_t w = bload96(vt, off);
            R.v[0].x = w.x;
            R.v[0].y = w.y;
            R.v[0].z = w.z;
          }
        }
        if (tid < (1 + C::NB) * kTile) {
          const uint32_t lr = local(tid & (kTile - 1));
          const int nb = tid / kTile - 1;
          R.s = __builtin_bit_cast(float, bload32(nb < 0 ? kst : vst, nb < 0 ? lr * 4u : (lr * C::NB + nb) * 4u));
        }
        return;
      }
#pragma unroll
      for (int i = 0; i < C::LOADS; ++i) {
        const int ch = tid + i * C::THREADS;
        if (ch < C::CHUNKS) {
          const int tt = ch / (D / 16), part = ch % (D / 16);
          const uint32_t row = row_of(base + tt);
          R.k[i] = bload128(kc, row * (uint32_t)D + (uint32_t)part * 16u);
          if constexpr (!K8V3) R.v[i] = bload128(vc, row * (uint32_t)D + (uint32_t)part * 16u);
        }
      }
      if constexpr (K8V3) {
        if (tid < C::VJOBS) {
          const int grp = tid / C::SPLIT;
          const int tt = grp / C::NG, gi = grp % C::NG;
          const uint32_t off = row_of(base + tt) * (uint32_t)(C::WORDS * 4) + (uint32_t)gi * 12u;
          const u32x3_t w = bload96(vc, off);
          R.v[0].x = w.x;
          R.v[0].y = w.y;
          R.v[0].z = w.z;
        }
      }
      if (tid < (1 + C::NB) * kTile) {  // k_scale of key tid, then block (tid/32 - 1)'s V scale
        const uint32_t row = row_of(base + (tid & (kTile - 1)));
        if constexpr (C::NB == 1) {
          R.s = __builtin_bit_cast(float, bload32(tid < kTile ? ks : vs, row * 4u));
        } else {
          const int nb = tid / kTile - 1;
          R.s = __builtin_bit_cast(float, bload32(nb < 0 ? ks : vs, nb < 0 ? row * 4u : (row * C::NB + nb) * 4u));
        }
      }
    };
    // Window verify with fresh drafts: whether the tile at `base` holds
    // draft keys (wave-uniform), whose K then has a low fp16 part.
    auto fresh_tile = [&](int base) -> bool {
      if constexpr (WIN && !DENSE) return a.kd != nullptr && base + kTile > prefix && base < prefix + nq;
      return false;
    };
    // registers -> LDS buffer, converting int8 to fp16.  With fresh drafts
    // (WIN and a.kd set), the rows of draft keys take the drafts' fp16 K / V
    // and unit scales instead.
    auto store_tile = [&](const TileRegs& R, int buf, int base) {
      char* kb = smem + buf * C::BUF;
      char* vb = kb + C::KBYTES;
      float* sb = reinterpret_cast<float*>(vb + C::VBYTES);
      // draft index of tile key tt, or -1 when it is a prefix key / not fresh
      auto fresh_draft = [&](int tt) -> int {
        if constexpr (WIN && !DENSE) {
          const int di = base + tt - prefix;
          return (a.kd != nullptr && di >= 0 && di < nq) ? di : -1;
        }
        return -1;
      };
      if constexpr (DENSE) {
#pragma unroll
        for (int i = 0; i < C::LOADS_F16; ++i) {
          const int ch = tid + i * C::THREADS;
          if (ch < C::CHUNKS_F16) {
            const int tt = ch / (D / 8), part = ch % (D / 8);
            *reinterpret_cast<u32x4_t*>(kb + tt * C::KROW + part * 16) = R.k[i];
            *reinterpret_cast<u32x4_t*>(vb + vrow_of(tt) * C::VROW + part * 16) = R.v[i];
          }
        }
        // the K scale slots carry the softmax scale (q is unscaled), the V slots 1
        if (tid < 2 * kTile) sb[tid] = tid < kTile ? a.qscale : R.s;
        return;
      }
#pragma unroll
      for (int i = 0; i < C::LOADS; ++i) {
        const int ch = tid + i * C::THREADS;
        if (ch < C::CHUNKS) {
          const int tt = ch / (D / 16), part = ch % (D / 16);
          const int di = fresh_draft(tt);
          half8_t k0, k1, v0, v1;
          if (di >= 0) {  // the draft's fresh values, dims part*16 .. +16: K as fp16 hi (+ lo below)
            const float* kp = a.kd + (int64_t)b * a.kd_stride_b + (int64_t)di * a.kd_stride_s +
                              (int64_t)h * a.kd_stride_h + part * 16;
            const _Float16* vp = a.vd + (int64_t)b * a.vd_stride_b + (int64_t)di * a.vd_stride_s +
                                 (int64_t)h * a.vd_stride_h + part * 16;
            half8_t l0, l1;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float x0 = kp[e], x1 = kp[8 + e];
              k0[e] = (_Float16)x0;
              k1[e] = (_Float16)x1;
              l0[e] = (_Float16)(x0 - (float)k0[e]);
              l1[e] = (_Float16)(x1 - (float)k1[e]);
            }
            char* klo = smem + C::KLO_OFF + buf * C::KBYTES + tt * C::KROW + part * 32;
            *reinterpret_cast<half8_t*>(klo) = l0;
            *reinterpret_cast<half8_t*>(klo + 16) = l1;
            v0 = *reinterpret_cast<const half8_t*>(vp);
            v1 = *reinterpret_cast<const half8_t*>(vp + 8);
          } else {
            if constexpr (WIN && !DENSE) {
              if (fresh_tile(base)) {  // a prefix key in a tile holding drafts: no low part
                char* klo = smem + C::KLO_OFF + buf * C::KBYTES + tt * C::KROW + part * 32;
                *reinterpret_cast<half8_t*>(klo) = half8_t{};
                *reinterpret_cast<half8_t*>(klo + 16) = half8_t{};
              }
            }
            k0 = i8x8_to_f16(u32x2_t{R.k[i].x, R.k[i].y});
            k1 = i8x8_to_f16(u32x2_t{R.k[i].z, R.k[i].w});
            if constexpr (!K8V3) {
              v0 = i8x8_to_f16(u32x2_t{R.v[i].x, R.v[i].y});
              v1 = i8x8_to_f16(u32x2_t{R.v[i].z, R.v[i].w});
            }
          }
          *reinterpret_cast<half8_t*>(kb + tt * C::KROW + part * 32) = k0;
          *reinterpret_cast<half8_t*>(kb + tt * C::KROW + part * 32 + 16) = k1;
          if (!K8V3 || di >= 0) {  // K8V3: prefix V rows come from the code expansion below
            *reinterpret_cast<half8_t*>(vb + vrow_of(tt) * C::VROW + part * 32) = v0;
            *reinterpret_cast<half8_t*>(vb + vrow_of(tt) * C::VROW + part * 32 + 16) = v1;
          }
        }
      }
      if constexpr (K8V3) {  // 32 / SPLIT codes of one group -> fp16 codebook entries
        if (tid < C::VJOBS && fresh_draft((tid / C::SPLIT) / C::NG) < 0) {
          const int grp = tid / C::SPLIT, part = tid % C::SPLIT;  // part: which 32 / SPLIT values
          const int tt = grp / C::NG, gi = grp % C::NG;
          const int sh = part * (32 / C::SPLIT);
          const uint32_t w0 = R.v[0].x >> sh, w1 = R.v[0].y >> sh, w2 = R.v[0].z >> sh;
          char* dst = vb + vrow_of(tt) * C::VROW + gi * 64 + sh * 2;
#pragma unroll
          for (int q4 = 0; q4 < 8 / C::SPLIT; q4 += 2) {
            u32x4_t o;
            const uint32_t sel0 = spread4(w0 >> (4 * q4)) | (spread4(w1 >> (4 * q4)) << 1) | (spread4(w2 >> (4 *
            q4)) << 2);
            const uint32_t sel1 = spread4(w0 >> (4 * q4 + 4)) | (spread4(w1 >> (4 * q4 + 4)) << 1) |
                                  (spread4(w2 >> (4 * q4 + 4)) << 2);
            const u32x2_t r0 = codebook_lookup4(sel0, tlo03, tlo47, thi03, thi47);
            const u32x2_t r1 = codebook_lookup4(sel1, tlo03, tlo47, thi03, thi47);
            o.x = r0.x; o.y = r0.y; o.z = r1.x; o.w = r1.y;
            *reinterpret_cast<u32x4_t*>(dst + q4 * 8) = o;
          }
        }
      }
      if (tid < (1 + C::NB) * kTile) sb[tid] = fresh_draft(tid & (kTile - 1)) >= 0 ? 1.0f : R.s;
    };

    // ---- one 32-key tile from LDS buffer `buf` ----
    auto process = [&](int buf, int base, auto masked_tag) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      const char* kb = smem + buf * C::BUF;
      const char* vb = kb + C::KBYTES;
      const float* sb = reinterpret_cast<const float*>(vb + C::VBYTES);
      // QK: each K operand read from LDS feeds the MFMAs of every row group
      float4_t sc[RG][2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float4_t cacc[RG];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) cacc[rg] = float4_t{0.f, 0.f, 0.f, 0.f};
        const char* krow = kb + (16 * s + c) * C::KROW + g * C::KCH * 2;
#pragma unroll
        for (int m = 0; m < C::NQK; ++m) {
          const half8_t ka = *reinterpret_cast<const half8_t*>(krow + 16 * m);
#pragma unroll
          for (int rg = 0; rg < RG; ++rg) {
            cacc[rg] = mfma16x16x32(ka, qhi[rg][m], cacc[rg]);
            if constexpr (!DENSE) cacc[rg] = mfma16x16x32(ka, qlo[rg][m], cacc[rg]);
          }
        }
        if constexpr (WIN && !DENSE) {  // fresh draft keys: K = hi + lo (masked or not)
          if (fresh_tile(base)) {
            const char* lrow = smem + C::KLO_OFF + buf * C::KBYTES + (16 * s + c) * C::KROW + g * C::KCH * 2;
#pragma unroll
            for (int m = 0; m < C::NQK; ++m) {
              const half8_t kl = *reinterpret_cast<const half8_t*>(lrow + 16 * m);
#pragma unroll
              for (int rg = 0; rg < RG; ++rg) cacc[rg] = mfma16x16x32(kl, qhi[rg][m], cacc[rg]);
            }
          }
        }
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) sc[rg][s] = cacc[rg];
      }
      // dense inputs: the softmax runs at raised wave priority, so the other
      // wave of the SIMD issues its MFMAs around it (+1.6 %; the paged
      // instantiations gain nothing or lose up to 3 % with it)
      constexpr bool prio = DENSE;
      if constexpr (prio) __builtin_amdgcn_s_setprio(1);
      float4_t ksc[2], vsc[2], vsc1[2];  // vsc1: K8V3 head_dim 256, the second block's norms
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        ksc[s] = *reinterpret_cast<const float4_t*>(sb + 16 * s + 4 * g);
        vsc[s] = *reinterpret_cast<const float4_t*>(sb + kTile + 16 * s + 4 * g);
        if constexpr (C::NB == 2) vsc1[s] = *reinterpret_cast<const float4_t*>(sb + 2 * kTile + 16 * s + 4 * g);
      }
      // Rescales are rare: a V scale above the bound lowers esh (WeightShift),
      // a tile max past the running max by more than the slack raises it.
      // Both are decided first, and the rest of the tile (weights, PV) is
      // instantiated with and without the rescale: as a branch inside one
      // instance, the compiler copied every accumulator register on the
      // common path to merge the two.  For the V-scale test each lane checks
      // one of the tile's (1 + NB) * 32 staged scales -- lane (g, c) the scale
      // of key 16 ((c >> 2) & 1) + 4 g + (c & 3), of block c >> 3 when there
      // are two -- so the 64 lanes cover them all.
      // (dense inputs: unit scales, the shift set once before the key loop)
      const int pk = 16 * ((c >> 2) & 1) + 4 * g + (c & 3);
      float vp = DENSE ? 0.0f : sb[kTile * (1 + ((c >> 3) & (C::NB - 1))) + pk];
      if constexpr (MASKED && WIN && !DENSE) vp = base + pk >= lo_key ? vp : 0.0f;  // below the window: any value
      auto shift_weights = [&]() {
        if (__builtin_amdgcn_ballot_w64(vp > ws.vbound()) == 0) return;
        float vmx = fmaxf(vp, shfl_xor_f(vp, 1));
        vmx = fmaxf(vmx, shfl_xor_f(vmx, 2));
        vmx = fmaxf(vmx, shfl_xor_f(vmx, 4));
        vmx = fmaxf(vmx, shfl_xor_f(vmx, 8));
        const int d = ws.raise(max_x32(max_x16(vmx)), kMaxSlack);
        const float f = __builtin_ldexpf(1.0f, d);
#pragma unroll
        for (int r = 0; r < RG; ++r) {
          l_run[r] *= f;
#pragma unroll
          for (int n = 0; n < C::NPV; ++n) acc[r][n] *= f;
          m_ref[r] -= (float)d;
        }
      };
      // key kk of the tile visible to this lane's row of group rg (MASKED only)
      auto visible = [&](int rg, int s, int i) -> bool {
        const int kk = base + 16 * s + 4 * g + i;
        const int di = kk - prefix;  // draft index when >= 0
        bool vis = kk < kv_end && row_live[rg] && (!WIN || kk >= (DENSE ? prefix + pos[rg] - a.window : lo_key));
        if (di >= 0) vis = vis && (tree ? (di < 64 && ((tmask[rg] >> di) & 1ull)) : di <= pos[rg]);
        return vis;
      };
      float y[RG][2][4];  // score relative to the running max, log2 domain
      bool any = false;   // some row group (or the V-scale bound) needs a rescale
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        float my = kNegInf;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = __builtin_fmaf(sc[rg][s][i], ksc[s][i], -m_ref[rg]);
            if constexpr (MASKED) v = visible(rg, s, i) ? v : kNegInf;
            y[rg][s][i] = v;
            my = fmaxf(my, v);
          }
        }
        my = max_x16(my);
        my = max_x32(my);
        any = any || __builtin_amdgcn_ballot_w64(my > ws.thr() || (rg == 0 && vp > ws.vbound())) != 0;
      }
      auto tail = [&](auto resc_tag) {
        constexpr bool RESC = decltype(resc_tag)::value;
        if constexpr (RESC) {
          shift_weights();
#pragma unroll
          for (int rg = 0; rg < RG; ++rg) {
            // raise the running max to the tile's (from the products, exactly;
            // every row group, also one within the slack), rescale, and take
            // the scores relative to the new max
            float mt = kNegInf;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                float x = sc[rg][s][i] * ksc[s][i];
                if constexpr (MASKED) x = visible(rg, s, i) ? x : kNegInf;
                mt = fmaxf(mt, x);
              }
            }
            mt = max_x16(mt);
            mt = max_x32(mt);
            const float m_new = fmaxf(m_ref[rg], mt - (float)ws.esh);
            const float alpha = __builtin_amdgcn_exp2f(m_ref[rg] - m_new);
            l_run[rg] *= alpha;
#pragma unroll
            for (int n = 0; n < C::NPV; ++n) acc[rg][n] *= alpha;
            m_ref[rg] = m_new;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                float v = __builtin_fmaf(sc[rg][s][i], ksc[s][i], -m_new);
                if constexpr (MASKED) v = visible(rg, s, i) ? v : kNegInf;
                y[rg][s][i] = v;
              }
            }
          }
        }
        half8_t pbh[RG], pbl[RG], pbh1[RG], pbl1[RG];  // B of the PV MFMAs (pbh1 / pbl1: the second V block)
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
          // weights p * (V scale | block norm) as fp16 hi + lo: hi keeps the
          // weight's top 11 significant bits (exact in fp16 for weights in
          // fp16's normal range), lo the exact fp32 rest
          float wh[2][4], wl[2][4], wh1[2][4], wl1[2][4];
#pragma unroll
          for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float e = __builtin_amdgcn_exp2f(y[rg][s][i]);  // 0 for masked keys
              l_run[rg] += e;
              // masked keys: e = 0, but their scale (past the visible keys, or
              // below a window) may be any value, inf and NaN included
              // (materialized: hi and lo must both come from this one fp32 value,
              // not from a product the compiler contracts into the lo subtraction)
              float w = materialize(e * vsc[s][i]);
              if constexpr (MASKED) w = (y[rg][s][i] != kNegInf) ? w : 0.0f;
              wh[s][i] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w) & 0xFFFFE000u);
              wl[s][i] = w - wh[s][i];
              if constexpr (C::NB == 2) {
                float w1 = materialize(e * vsc1[s][i]);
                if constexpr (MASKED) w1 = (y[rg][s][i] != kNegInf) ? w1 : 0.0f;
                wh1[s][i] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, w1) & 0xFFFFE000u);
                wl1[s][i] = w1 - wh1[s][i];
              }
            }
          }
#pragma unroll
          for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
              const half2_t h2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(wh[s][i], wh[s][i + 1]));
              const half2_t l2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(wl[s][i], wl[s][i + 1]));
              pbh[rg][4 * s + i] = h2[0];
              pbh[rg][4 * s + i + 1] = h2[1];
              pbl[rg][4 * s + i] = l2[0];
              pbl[rg][4 * s + i + 1] = l2[1];
              if constexpr (C::NB == 2) {
                const half2_t h21 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(wh1[s][i], wh1[s][i + 1]));
                const half2_t l21 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(wl1[s][i], wl1[s][i + 1]));
                pbh1[rg][4 * s + i] = h21[0];
                pbh1[rg][4 * s + i + 1] = h21[1];
                pbl1[rg][4 * s + i] = l21[0];
                pbl1[rg][4 * s + i + 1] = l21[1];
              }
            }
          }
        }
        if constexpr (prio) __builtin_amdgcn_s_setprio(0);
        // PV: each V^T operand read from LDS feeds the MFMAs of every row group
#pragma unroll
        for (int n = 0; n < C::NPV; ++n) {
          const int r0 = 8 * g + ((lane >> 2) & 3);
          const int colb = (16 * n + 4 * (lane & 3)) * 2;
          const i16x4_t lw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((S8KV_LDS i16x4_t*)(vb + r0 * C::VROW + colb));
          const i16x4_t hw =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((S8KV_LDS i16x4_t*)(vb + (r0 + 4) * C::VROW + colb));
          const half4_t l4 = __builtin_bit_cast(half4_t, lw), h4 = __builtin_bit_cast(half4_t, hw);
          const half8_t va = half8_t{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
          const bool second = C::NB == 2 && 16 * n >= 128;  // dims 128..255 of a K8V3 head_dim-256 key
#pragma unroll
          for (int rg = 0; rg < RG; ++rg) {
            acc[rg][n] = mfma16x16x32(va, second ? pbh1[rg] : pbh[rg], acc[rg][n]);
            acc[rg][n] = mfma16x16x32(va, second ? pbl1[rg] : pbl[rg], acc[rg][n]);
          }
        }
      };
      if (any)
        tail(std::true_type{});
      else
        tail(std::false_type{});
    };

    // Tiles alternate between two LDS buffers; their global loads are issued
    // two tiles ahead into two register sets (A for even tiles, B for odd),
    // so a load has two tiles of compute to arrive.
    auto compute = [&](int buf, int base) {
      // a tile needs masking when it reaches keys that some row of the block
      // does not see, or the end of the visible keys (wave-uniform: MFMAs must
      // run with every lane active; rows past the query count are zeroed at the
      // end instead)
      if (base + kTile <= vis_all && base + kTile <= kv_end && (!WIN || base >= lo_all))
        process(buf, base, std::false_type{});
      else
        process(buf, base, std::true_type{});
    };
    const int ntiles = (u1 - u0 + kTile - 1) / kTile;
    TileRegs ra, rb;
    load_tile(ra, u0);
    if (ntiles > 1) load_tile(rb, u0 + kTile);
    store_tile(ra, 0, u0);
    __syncthreads();
    for (int t = 0; t < ntiles; t += 2) {
      const int base = u0 + t * kTile;
      if (t + 2 < ntiles) load_tile(ra, base + 2 * kTile);
      compute(0, base);
      if (t + 1 < ntiles) store_tile(rb, 1, base + kTile);
      __syncthreads();
      if (t + 1 >= ntiles) break;
      if (t + 3 < ntiles) load_tile(rb, base + 3 * kTile);
      compute(1, base + kTile);
      if (t + 2 < ntiles) store_tile(ra, 0, base + 2 * kTile);
      __syncthreads();
    }
  }

  // ---- split: this wave's unnormalized rows to the partials ----
  if (a.splits > 1) {
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
      const float l_tot = sum_x32(sum_x16(l_run[rg]));
      const int rl = (rg * C::WAVES + wave) * 16 + c;  // row within the block
      float* pr = a.part + ((((int64_t)p * a.n_qblocks + qb) * a.splits + sp) * C::ROWS + rl) * (D + 4);
#pragma unroll
      for (int n = 0; n < C::NPV; ++n) *reinterpret_cast<float4_t*>(pr + 16 * n + 4 * g) = acc[rg][n];
      if (g == 0) {
        pr[D] = m_ref[rg];
        pr[D + 1] = l_tot;
      }
    }
    return;
  }

  // ---- normalize and write this wave's rows ----
#pragma unroll
  for (int rg = 0; rg < RG; ++rg) {
    const float l_tot = sum_x32(sum_x16(l_run[rg]));
    // (dense: only the sequence's own query tokens -- the next ones belong to the next sequence)
    if (DENSE ? row_live[rg] : pos[rg] < a.max_queries) {
      const float inv = (row_live[rg] && l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
      _Float16* op = DENSE ? a.out + (int64_t)(q0 + pos[rg]) * a.o_stride_t + (int64_t)head[rg] * a.o_stride_h
                           : a.out + (((int64_t)b * a.num_q_heads + head[rg]) * a.max_queries + pos[rg]) * D;
#pragma unroll
      for (int n = 0; n < C::NPV; ++n) {
        half4_t o;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) o[rr] = (_Float16)(acc[rg][n][rr] * inv);
        *reinterpret_cast<half4_t*>(op + 16 * n + 4 * g) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wide verify (head_dim 128, paged int8 or K8V3 cache): 32 query rows per wave
// on v_mfma_f32_32x32x16_f16, so every K and V operand a wave reads from LDS
// feeds twice the MFMAs of a 16-row wave.  Lane (j = lane % 32, hf = lane /
// 32) holds query row j of its wave:
//   QK  : S^T[key][row] with A = K rows from LDS (key lane % 32, dims 64 hf ..
//         64 hf + 63, 8 per MFMA), B = the rotated, pre-scaled q of row j over
//         the same dims as fp16 hi + lo; lane l's result register r is key
//         8 (r / 4) + 4 hf + r % 4 of row j, so the softmax state of a row
//         lives in one lane pair (lane, lane ^ 32).
//   PV  : O^T[dim][row], A = V^T through ds_read_b64_tr_b16 from a plain
//         row-major fp16 V tile, B = the weights of the lane's own keys --
//         k-step t uses result registers 8t .. 8t + 7, whose keys are the
//         sixteen 16t + 8 (e / 4) + 4 hf + e % 4 that the transpose reads
//         deliver (rows 16t + 4 hf + 0..3 and 16t + 8 + 4 hf + 0..3).
// Numerics are the 16-row kernel's: the same q rotation and hi + lo split,
// the same lazy-max online softmax and hi + lo weights; only the order of
// the fp32 sums differs.
// ---------------------------------------------------------------------------
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// Two fp32 weights as fp16 hi + lo pairs: hi = w rounded toward zero to fp16
// (its top 11 significant bits in fp16's normal range), lo = w - hi exactly
// (v_fma_mix_f32 reads hi as fp16 out of the packed register), then rounded
// toward zero to fp16.  The asm reads only results of ordinary VALU
// instructions (no transcendental or MFMA result, whose wait states the
// compiler inserts for its own instructions only), and the rounded w it
// takes cannot be contracted into the subtraction.
__device__ __forceinline__ void split_pair(float w0, float w1, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(w0, w1));
  float l0, l1;
  asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(l0) : "v"(hi), "v"(w0));
  asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(l1) : "v"(hi), "v"(w1));
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(l0, l1));
}

template <bool K8V3, bool EIGHT>
struct WideCfg {
  static constexpr int D = 128;
  // EIGHT (calls with more than 128 query rows per sequence and KV head):
  // 8 waves (256 rows) per workgroup, one workgroup per CU, so twice the rows
  // share each tile's staging (K8V3: code expansion); else 4 waves, two per CU
  static constexpr int WAVES = EIGHT ? 8 : 4;
  static constexpr int WG_PER_CU = 8 / WAVES;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int ROWS = 32 * WAVES;  // query rows per workgroup
  static constexpr int KROW = 2 * D + 16;  // LDS pitch of an fp16 K row (8 consecutive rows: distinct 16-byte slots)
  static constexpr int VROW = 2 * D + 32;  // LDS pitch of an fp16 V row (4 rows of a transpose read: distinct banks)
  static constexpr int KBYTES = kTile * KROW;
  static constexpr int VBYTES = kTile * VROW;
  static constexpr int SBYTES = 2 * kTile * 4;  // k_scale, then the V scale (int8) or block norm (K8V3) per key
  static constexpr int BUF = KBYTES + VBYTES + SBYTES;
  static constexpr int CHUNKS = kTile * D / 16;  // 16-byte int8 chunks per K (or V) tile: one per thread
  static_assert(CHUNKS == 256, "one K chunk per thread of the first 256 (and one V chunk per thread of the last)");
  static constexpr int NG = D / 32;      // K8V3: 32-value code groups per key
  static constexpr int WORDS = 3 * NG;   // K8V3: packed words per key
  static constexpr int VJOBS = 2 * kTile * NG;  // K8V3: two threads per code group (16 values each)
  static_assert(VJOBS == 256, "one K8V3 expansion job per thread of the last 256");
  static constexpr int SMEM = 2 * BUF + kMaxSubBlocks * 4;
  // window verify with fresh drafts: the low fp16 part of the drafts' K per buffer
  static constexpr int KLO_OFF = (SMEM + 15) / 16 * 16;
  static constexpr int SMEM_WIN = KLO_OFF + 2 * KBYTES;
};

// DENSE: fresh fp16 K / V (attn_varlen), token-major with cu_seqlens, not
// rotated: q is the exact fp16 input (one QK MFMA per fragment) and the
// softmax scale multiplies the fp32 score through the staged K scales.
// WIN, dense: a band -- query s sees keys j >= prefix + s - window; paged:
// every row sees the last `window` prefix keys and the drafts, keys j >=
// prefix - window, the drafts' K / V from the cache or (FRESH, a.kd set) from
// the fresh fp32 K (rotated) and fp16 V rows of the drafts.
template <bool K8V3, bool DENSE = false, bool WIN = false, bool FRESH = false, bool EIGHT = false>
__global__ __launch_bounds__((WideCfg<K8V3, EIGHT>::THREADS), (WideCfg<K8V3, EIGHT>::WG_PER_CU)) void verify_wide_kernel(
    VerifyArgs a) {
  static_assert(!(DENSE && K8V3), "dense inputs: fp16 K / V");
  static_assert(!FRESH || (WIN && !DENSE), "fresh drafts: a paged window verify");
  using C = WideCfg<K8V3, EIGHT>;
  constexpr int D = C::D;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int* bt_lds = reinterpret_cast<int*>(smem + 2 * C::BUF);

  // workgroups of one (sequence, KV head) pair share an XCD (and its L2)
  const int P = a.batch * a.num_kv_heads;
  const int xcd = blockIdx.x & 7;
  const int rest = blockIdx.x >> 3;
  const int qb = rest % a.n_qblocks;
  const int rest2 = rest / a.n_qblocks;
  const int sp = rest2 % a.splits;
  const int p = (rest2 / a.splits) * 8 + xcd;
  if (p >= P) return;
  const int b = p / a.num_kv_heads;
  const int h = p - b * a.num_kv_heads;
  const int G = a.group;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31;  // this lane's query row within the wave (and the K row of its QK A operand)
  const int hf = lane >> 5;

  // dense: sequence b's queries are tokens cu_q[b] .., its keys cu_k[b] ..;
  // causal is bottom-right aligned (query s sees keys j <= s + nk - nq, which
  // may be none), else every key is visible
  int nq, prefix, nk = 0, q0 = 0, k0 = 0;
  if constexpr (DENSE) {
    q0 = a.cu_q[b];
    k0 = a.cu_k[b];
    const int nq_seq = max(0, a.cu_q[b + 1] - q0);
    nk = max(0, a.cu_k[b + 1] - k0);
    nq = min(nq_seq, a.max_queries);
    prefix = a.causal ? nk - nq_seq : nk;
  } else {
    nq = a.query_lens ? max(0, min(a.query_lens[b], a.max_queries)) : a.max_queries;
    prefix = max(0, a.prefix_lens[b]);
  }
  const int row0 = qb * C::ROWS;
  const int pos_hi = min(nq, (row0 + C::ROWS + G - 1) / G);
  const bool tree = a.tree_mask != nullptr;
  int kv_end = prefix + (tree ? nq : pos_hi);
  kv_end = min(kv_end, DENSE ? nk : a.max_context_len);
  if (row0 / G >= nq) kv_end = 0;
  const int vis_all = tree ? prefix : prefix + row0 / G + 1;
  // window: keys below lo_key are hidden from every row of the block (the key
  // loop starts at the tile holding it), keys from lo_all on from none
  const int lo_key = WIN ? max(0, prefix + (DENSE ? row0 / G : 0) - a.window) : 0;
  const int lo_all = WIN && DENSE ? prefix + min(nq - 1, (row0 + C::ROWS - 1) / G) - a.window : lo_key;

  const int r = row0 + wave * 32 + j;
  const int pos = r / G;
  const int head = h * G + (r - pos * G);
  const bool row_live = pos < nq;
  const uint64_t tmask = (tree && row_live) ? (uint64_t)a.tree_mask[(int64_t)b * a.max_queries + pos] : 0ull;

  // ---- q: rotate (FWHT over dims 64 hf .. 64 hf + 63 in-lane, then across
  // the lane pair), pre-scale, split into fp16 hi + lo; dense: the fp16 input ----
  half8_t qhi[8], qlo[DENSE ? 1 : 8];
  if constexpr (DENSE) {
    const _Float16* qp = a.q + (int64_t)q0 * a.q_stride_s + (int64_t)head * a.q_stride_h +
                         (int64_t)(row_live ? pos : 0) * a.q_stride_s + hf * 64;
#pragma unroll
    for (int m = 0; m < 8; ++m) qhi[m] = row_live ? *reinterpret_cast<const half8_t*>(qp + 8 * m) : half8_t{};
  } else {
    float x[64];
    const _Float16* qp = a.q + (int64_t)b * a.q_stride_b + (int64_t)head * a.q_stride_h +
                         (int64_t)(row_live ? pos : 0) * a.q_stride_s + hf * 64;
#pragma unroll
    for (int i = 0; i < 64; i += 8) {
      const half8_t v = *reinterpret_cast<const half8_t*>(qp + i);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[i + e] = row_live ? (float)v[e] : 0.0f;
    }
#pragma unroll
    for (int hs = 1; hs < 64; hs <<= 1) {
#pragma unroll
      for (int i = 0; i < 64; ++i) {
        if ((i & hs) == 0) {
          const float x0 = x[i], x1 = x[i + hs];
          x[i] = x0 + x1;
          x[i + hs] = x0 - x1;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 64; ++i) x[i] = butterfly_x32(x[i], lane);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // (materialized: hi and lo must both come from this one fp32 value)
        const float val = materialize(x[8 * m + e] * a.qscale);
        const _Float16 qh = (_Float16)val;
        qhi[m][e] = qh;
        qlo[m][e] = (_Float16)(val - (float)qh);
      }
    }
  }

  float m_ref = kMaxInit, l_run = 0.0f;
  float16_t acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) acc[n] = float16_t{};
  WeightShift ws(kMaxSlack);
  if constexpr (DENSE) ws.raise(1.0f, kMaxSlack);  // fp16 K / V: every V scale is 1

  const rsrc_t kc = make_rsrc(a.k_cache, a.kc_bytes);
  const rsrc_t vc = make_rsrc(a.v_cache, a.vc_bytes);
  const rsrc_t ks = make_rsrc(a.k_scale, a.ks_bytes);
  const rsrc_t vs = make_rsrc(a.v_scale, a.vs_bytes);
  uint32_t tlo03 = 0, tlo47 = 0, thi03 = 0, thi47 = 0;
  if constexpr (K8V3) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t hb = __builtin_bit_cast(uint16_t, (_Float16)a.v_codebook[i]);
      const uint32_t lw = hb & 0xFFu, hw = hb >> 8;
      if (i < 4) { tlo03 |= lw << (8 * i); thi03 |= hw << (8 * i); }
      else { tlo47 |= lw << (8 * (i - 4)); thi47 |= hw << (8 * (i - 4)); }
    }
  }
  const int bs_log2 = a.bs_log2;
  const uint32_t bsm = (1u << bs_log2) - 1u;
  const uint32_t hkv = (uint32_t)a.num_kv_heads;
  const int32_t* bt_row = a.block_table + (int64_t)b * a.bt_stride;

  // this workgroup's keys: split sp of the block's tile-aligned key range
  int k_lo = lo_key & ~(kTile - 1), k_hi = kv_end;
  if (a.splits > 1) {
    const int chunk = ((max(0, kv_end - k_lo) + a.splits - 1) / a.splits + kTile - 1) & ~(kTile - 1);
    k_lo += sp * chunk;
    k_hi = min(kv_end, k_lo + chunk);
  }
  // A wave whose 32 rows are all past the query count (a short draft tree,
  // the last block of a chunk) takes part in the tile loads, conversions and
  // barriers only; its rows are written as zeros.  The key loop is
  // instantiated for both kinds of wave, so neither carries the other's branch.
  const bool wave_live = (row0 + wave * 32) / G < nq;
  auto key_loop = [&](auto live_tag) {
  constexpr bool LIVE = decltype(live_tag)::value;
  for (int u0 = k_lo; u0 < k_hi; u0 += kSubKeys) {
    const int u1 = min(k_hi, u0 + kSubKeys);
    const int fb = u0 >> bs_log2;
    const int nblk = ((u1 - 1) >> bs_log2) - fb + 1;
    __syncthreads();  // previous users of bt_lds and the tile buffers are done
    if constexpr (!DENSE)
      for (int i = tid; i < nblk; i += C::THREADS) bt_lds[i] = bt_row[fb + i];
    __syncthreads();

    auto row_of = [&](int kk) -> uint32_t {
      kk = min(kk, u1 - 1);
      const uint32_t blk = (uint32_t)bt_lds[(kk >> bs_log2) - fb];
      return ((blk * hkv + (uint32_t)h) << bs_log2) + ((uint32_t)kk & bsm);
    };

    // window verify with fresh drafts: whether the tile at `base` holds draft
    // keys (wave-uniform), whose K then has a low fp16 part, and the draft
    // index of its key tt (-1: a prefix key, or no fresh drafts)
    auto fresh_tile = [&](int base) -> bool {
      if constexpr (FRESH) return base + kTile > prefix && base < prefix + nq;
      return false;
    };
    auto fresh_draft = [&](int base, int tt) -> int {
      if constexpr (FRESH) {
        const int di = base + tt - prefix;
        return (di >= 0 && di < nq) ? di : -1;
      }
      return -1;
    };
    // dense: 512 16-byte fp16 K chunks and as many V chunks per tile, two
    // each per thread of a 4-wave workgroup, one of an 8-wave one
    constexpr int NCH = DENSE ? 512 / C::THREADS : 1;
    struct TileRegs {
      u32x4_t k[NCH], v[NCH];
      float s;
    };
    // one 16-byte K chunk and one V chunk (K8V3: a half code group's three
    // words) per thread, and the tile's 2 x 32 scales in threads 0..63
    // (the cache rows of fresh drafts are loaded too, and not used)
    auto load_tile = [&](TileRegs& R, int base) {
      if constexpr (DENSE) {  // fp16 rows of keys base .. base + 31 (clamped to the last key)
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          const int ch = tid + i * C::THREADS, tt = ch >> 4, part = ch & 15;
          const int64_t tok = k0 + min(base + tt, nk - 1);
          R.k[i] = *reinterpret_cast<const u32x4_t*>(a.k_f16 + tok * a.k_stride_t + h * a.k_stride_h + part * 8);
          R.v[i] = *reinterpret_cast<const u32x4_t*>(a.v_f16 + tok * a.v_stride_t + h * a.v_stride_h + part * 8);
        }
        R.s = 1.0f;
        return;
      }
      // 4 waves: every thread one K and one V chunk; 8 waves: threads 0..255
      // the K chunks, 256..511 the V chunks (vt: the V job index)
      constexpr bool SPLITKV = C::WAVES == 8;
      const bool kthr = !SPLITKV || tid < 256, vthr = !SPLITKV || tid >= 256;
      const int vt = tid & 255;
      const int tt = tid >> 3 & 31, part = tid & 7;
      const uint32_t row = row_of(base + tt);
      if (kthr) R.k[0] = bload128(kc, row * (uint32_t)D + (uint32_t)part * 16u);
      if (!vthr) {
      } else if constexpr (K8V3) {
        const int grp = vt >> 1;
        const int gt = grp / C::NG, gi = grp % C::NG;
        const uint32_t off = row_of(base + gt) * (uint32_t)(C::WORDS * 4) + (uint32_t)gi * 12u;
        const u32x3_t w = bload96(vc, off);
        R.v[0].x = w.x;
        R.v[0].y = w.y;
        R.v[0].z = w.z;
      } else {
        R.v[0] = bload128(vc, row * (uint32_t)D + (uint32_t)part * 16u);
      }
      // (two loads, each with one descriptor: a descriptor chosen per lane
      // would be issued lane by lane)
      if (tid < kTile) R.s = __builtin_bit_cast(float, bload32(ks, row_of(base + tid) * 4u));
      else if (tid < 2 * kTile) R.s = __builtin_bit_cast(float, bload32(vs, row_of(base + tid - kTile) * 4u));
    };
    auto store_tile = [&](const TileRegs& R, int buf, int base) {
      char* kb = smem + buf * C::BUF;
      char* vb = kb + C::KBYTES;
      float* sb = reinterpret_cast<float*>(vb + C::VBYTES);
      if constexpr (DENSE) {  // fp16 rows as they are; K "scales" carry the softmax scale, V scales are 1
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          const int ch = tid + i * C::THREADS, tt = ch >> 4, part = ch & 15;
          *reinterpret_cast<u32x4_t*>(kb + tt * C::KROW + part * 16) = R.k[i];
          *reinterpret_cast<u32x4_t*>(vb + tt * C::VROW + part * 16) = R.v[i];
        }
        if (tid < 2 * kTile) sb[tid] = tid < kTile ? a.qscale : 1.0f;
        return;
      }
      constexpr bool SPLITKV = C::WAVES == 8;
      const bool kthr = !SPLITKV || tid < 256, vthr = !SPLITKV || tid >= 256;
      const int vt = tid & 255;
      const int tt = tid >> 3 & 31, part = tid & 7;
      const int di = kthr ? fresh_draft(base, tt) : -1;
      if (!kthr) {
      } else if (di >= 0) {  // the draft's fresh values, dims part*16 .. +16: K as fp16 hi + lo, V as it is
        const float4_t* kp = reinterpret_cast<const float4_t*>(
            a.kd + (int64_t)b * a.kd_stride_b + (int64_t)di * a.kd_stride_s + (int64_t)h * a.kd_stride_h + part * 16);
        const _Float16* vp = a.vd + (int64_t)b * a.vd_stride_b + (int64_t)di * a.vd_stride_s +
                             (int64_t)h * a.vd_stride_h + part * 16;
        const float4_t kx[4] = {kp[0], kp[1], kp[2], kp[3]};  // (rows 16-byte aligned: checked on the host)
        half8_t k0, k1, l0, l1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x0 = kx[e >> 2][e & 3], x1 = kx[2 + (e >> 2)][e & 3];
          k0[e] = (_Float16)x0;
          k1[e] = (_Float16)x1;
          l0[e] = (_Float16)(x0 - (float)k0[e]);
          l1[e] = (_Float16)(x1 - (float)k1[e]);
        }
        char* klo = smem + C::KLO_OFF + buf * C::KBYTES + tt * C::KROW + part * 32;
        *reinterpret_cast<half8_t*>(klo) = l0;
        *reinterpret_cast<half8_t*>(klo + 16) = l1;
        *reinterpret_cast<half8_t*>(kb + tt * C::KROW + part * 32) = k0;
        *reinterpret_cast<half8_t*>(kb + tt * C::KROW + part * 32 + 16) = k1;
        *reinterpret_cast<half8_t*>(vb + tt * C::VROW + part * 32) = *reinterpret_cast<const half8_t*>(vp);
        *reinterpret_cast<half8_t*>(vb + tt * C::VROW + part * 32 + 16) = *reinterpret_cast<const half8_t*>(vp + 8);
      } else {
        if (fresh_tile(base)) {  // a prefix key in a tile holding drafts: no low part
          char* klo = smem + C::KLO_OFF + buf * C::KBYTES + tt * C::KROW + part * 32;
          *reinterpret_cast<half8_t*>(klo) = half8_t{};
          *reinterpret_cast<half8_t*>(klo + 16) = half8_t{};
        }
        *reinterpret_cast<half8_t*>(kb + tt * C::KROW + part * 32) = i8x8_to_f16(u32x2_t{R.k[0].x, R.k[0].y});
        *reinterpret_cast<half8_t*>(kb + tt * C::KROW + part * 32 + 16) = i8x8_to_f16(u32x2_t{R.k[0].z, R.k[0].w});
      }
      // int8 V rows: by the V threads (the same key and part as a K thread's
      // tt, part; a fresh draft's V is written above with its K)
      if constexpr (!K8V3) {
        if (vthr && fresh_draft(base, tt) < 0) {
          *reinterpret_cast<half8_t*>(vb + tt * C::VROW + part * 32) = i8x8_to_f16(u32x2_t{R.v[0].x, R.v[0].y});
          *reinterpret_cast<half8_t*>(vb + tt * C::VROW + part * 32 + 16) = i8x8_to_f16(u32x2_t{R.v[0].z, R.v[0].w});
        }
      }
      if constexpr (K8V3) {  // 16 codes of one group -> fp16 codebook entries (prefix keys)
        const int grp = vt >> 1, half = vt & 1;
        const int gt = grp / C::NG, gi = grp % C::NG;
        if (vthr && fresh_draft(base, gt) < 0) {
          const int sh = half * 16;
          const uint32_t w0 = R.v[0].x >> sh, w1 = R.v[0].y >> sh, w2 = R.v[0].z >> sh;
          char* dst = vb + gt * C::VROW + gi * 64 + sh * 2;
#pragma unroll
          for (int q4 = 0; q4 < 4; q4 += 2) {
            u32x4_t o;
            const uint32_t sel0 =
                spread4(w0 >> (4 * q4)) | (spread4(w1 >> (4 * q4)) << 1) | (spread4(w2 >> (4 * q4)) << 2);
            const uint32_t sel1 = spread4(w0 >> (4 * q4 + 4)) | (spread4(w1 >> (4 * q4 + 4)) << 1) |
                                  (spread4(w2 >> (4 * q4 + 4)) << 2);
            const u32x2_t r0 = codebook_lookup4(sel0, tlo03, tlo47, thi03, thi47);
            const u32x2_t r1 = codebook_lookup4(sel1, tlo03, tlo47, thi03, thi47);
            o.x = r0.x; o.y = r0.y; o.z = r1.x; o.w = r1.y;
            *reinterpret_cast<u32x4_t*>(dst + q4 * 8) = o;
          }
        }
      }
      // a V scale is staged finite (NaN and inf -> 2^100): the weight of a
      // hidden key, exp2(-inf) * scale, is then 0 whatever was stored there
      // (clamped here, where the load is consumed, not where it is issued);
      // a fresh draft's K and V scales are 1
      if (tid < 2 * kTile)
        sb[tid] = fresh_draft(base, tid & (kTile - 1)) >= 0 ? 1.0f : tid < kTile ? R.s : fminf(R.s, 0x1p100f);
    };

    // ---- one 32-key tile from LDS buffer `buf` ----
    // Only the scores depend on the tile's kind (keys hidden from some row:
    // masked, as -inf); the rescale, the weights and the PV are one code path
    // for every tile, so the accumulators keep their registers throughout.
    auto process = [&](int buf, int base, bool masked) {
      const char* kb = smem + buf * C::BUF;
      const char* vb = kb + C::KBYTES;
      const float* sb = reinterpret_cast<const float*>(vb + C::VBYTES);
      float16_t sc = float16_t{};
      {
        const char* krow = kb + j * C::KROW + hf * 128;
        half8_t ka[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) ka[m] = *reinterpret_cast<const half8_t*>(krow + 16 * m);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          sc = mfma32x32x16(ka[m], qhi[m], sc);
          if constexpr (!DENSE) sc = mfma32x32x16(ka[m], qlo[m], sc);
        }
      }
      if constexpr (FRESH) {  // fresh draft keys: K = hi + lo
        if (fresh_tile(base)) {
          const char* lrow = smem + C::KLO_OFF + buf * C::KBYTES + j * C::KROW + hf * 128;
#pragma unroll
          for (int m = 0; m < 8; ++m) sc = mfma32x32x16(*reinterpret_cast<const half8_t*>(lrow + 16 * m), qhi[m], sc);
        }
      }
      // this lane's keys: register r is key 8 (r / 4) + 4 hf + r % 4
      float4_t ks4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) ks4[q] = *reinterpret_cast<const float4_t*>(sb + 8 * q + 4 * hf);
      auto kscale = [&](int rr) -> float { return ks4[rr >> 2][rr & 3]; };
      float y[16];  // score relative to the running max, log2 domain; -inf: hidden from this row
      if (masked) {
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const int kk = base + 8 * (rr >> 2) + 4 * hf + (rr & 3);
          const int di = kk - prefix;
          const bool dvis = tree ? ((uint32_t)di < 64u && ((tmask >> (di & 63)) & 1ull)) : di <= pos;
          const bool vis = kk < kv_end && row_live && (di < 0 || dvis) &&
                           (!WIN || kk >= (DENSE ? prefix + pos - a.window : lo_key));
          const float v = __builtin_fmaf(sc[rr], kscale(rr), -m_ref);
          y[rr] = vis ? v : kNegInf;
        }
      } else {
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) y[rr] = __builtin_fmaf(sc[rr], kscale(rr), -m_ref);
      }
      float my = y[0];
#pragma unroll
      for (int rr = 1; rr < 16; ++rr) my = fmaxf(my, y[rr]);
      my = max_x32(my);
      // V-scale bound test: lane l checks the V scale of key l % 32 (paged
      // window: not of the keys below it, which may hold anything)
      float vp = sb[kTile + j];
      if constexpr (WIN && !DENSE) vp = base + j >= lo_key ? vp : 0.0f;
      if (__builtin_amdgcn_ballot_w64(my > ws.thr() || vp > ws.vbound()) != 0) {
        // rare: a V scale above the bound lowers the weight shift (by d, a
        // power of two folded into alpha), or a score passes the lazy slack:
        // the running max rises to the tile's (from the products, exactly),
        // l and the accumulators are rescaled, the scores re-referenced
        int d = 0;
        if (__builtin_amdgcn_ballot_w64(vp > ws.vbound()) != 0) {
          float vmx = fmaxf(vp, shfl_xor_f(vp, 1));
          vmx = fmaxf(vmx, shfl_xor_f(vmx, 2));
          vmx = fmaxf(vmx, shfl_xor_f(vmx, 4));
          vmx = fmaxf(vmx, shfl_xor_f(vmx, 8));
          d = ws.raise(max_x16(vmx), kMaxSlack);
        }
        m_ref -= (float)d;
        float mt = kNegInf;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) mt = fmaxf(mt, y[rr] != kNegInf ? sc[rr] * kscale(rr) : kNegInf);
        mt = max_x32(mt);
        const float m_new = fmaxf(m_ref, mt - (float)ws.esh);
        const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new) * __builtin_ldexpf(1.0f, d);
        l_run *= alpha;
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[n] *= alpha;  // (plain VALU: its MFMA hazards are the compiler's)
        m_ref = m_new;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) y[rr] = y[rr] != kNegInf ? __builtin_fmaf(sc[rr], kscale(rr), -m_new) : kNegInf;
      }
      const int li = lane & 15;
      const char* vrow = vb + (4 * hf + (li >> 2)) * C::VROW + (16 * ((lane >> 4) & 1) + 4 * (li & 3)) * 2;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        // weights p * (V scale | block norm) of keys 16t .. 16t + 15 as fp16
        // hi + lo (hi: the top 11 significant bits, exact in fp16 over its
        // normal range; lo: the rest); hidden keys weigh 0 whatever their
        // scale (inf and NaN included)
        const float4_t vs0 = *reinterpret_cast<const float4_t*>(sb + kTile + 16 * t + 4 * hf);
        const float4_t vs1 = *reinterpret_cast<const float4_t*>(sb + kTile + 16 * t + 8 + 4 * hf);
        u32x4_t hi4, lo4;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float w[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int rr = 8 * t + e + u;
            const float ev = __builtin_amdgcn_exp2f(y[rr]);  // 0 for hidden keys
            l_run += ev;
            w[u] = ev * (e + u < 4 ? vs0[e + u] : vs1[e + u - 4]);  // (finite scales: 0 for hidden keys)
          }
          uint32_t hw, lw;
          split_pair(w[0], w[1], hw, lw);
          hi4[e / 2] = hw;
          lo4[e / 2] = lw;
        }
        const half8_t pbh = __builtin_bit_cast(half8_t, hi4), pbl = __builtin_bit_cast(half8_t, lo4);
        // PV: V^T operands by transpose reads; lane (li, group G) reads row
        // 16t + 4 hf + li / 4 (+ 8), dims 32 n + 16 (G & 1) + 4 (li % 4) .. + 3
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const char* src = vrow + 16 * t * C::VROW + 64 * n;
          const i16x4_t lw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((S8KV_LDS i16x4_t*)(src));
          const i16x4_t hw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((S8KV_LDS i16x4_t*)(src + 8 * C::VROW));
          const half4_t l4 = __builtin_bit_cast(half4_t, lw), h4 = __builtin_bit_cast(half4_t, hw);
          const half8_t va = half8_t{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
          acc[n] = mfma32x32x16(va, pbh, acc[n]);
          acc[n] = mfma32x32x16(va, pbl, acc[n]);
        }
      }
    };

    // a tile is masked when it reaches keys that some row of the block does
    // not see, or the end of the visible keys (wave-uniform)
    auto compute = [&](int buf, int base) {
      if constexpr (LIVE)
        process(buf, base, !(base + kTile <= vis_all && base + kTile <= kv_end && (!WIN || base >= lo_all)));
    };
    const int ntiles = (u1 - u0 + kTile - 1) / kTile;
    TileRegs ra, rb;
    load_tile(ra, u0);
    if (ntiles > 1) load_tile(rb, u0 + kTile);
    store_tile(ra, 0, u0);
    __syncthreads();
    for (int t = 0; t < ntiles; t += 2) {  // (one exit: the accumulators keep their registers)
      const int base = u0 + t * kTile;
      if (t + 2 < ntiles) load_tile(ra, base + 2 * kTile);
      compute(0, base);
      if (t + 1 < ntiles) store_tile(rb, 1, base + kTile);
      __syncthreads();
      if (t + 1 < ntiles) {
        if (t + 3 < ntiles) load_tile(rb, base + 3 * kTile);
        compute(1, base + kTile);
        if (t + 2 < ntiles) store_tile(ra, 0, base + 2 * kTile);
        __syncthreads();
      }
    }
  }
  };
  if (wave_live)
    key_loop(std::true_type{});
  else
    key_loop(std::false_type{});

  const float l_tot = sum_x32(l_run);
  // ---- split: this wave's unnormalized rows to the partials ----
  if (a.splits > 1) {
    const int rl = wave * 32 + j;
    float* pr = a.part + ((((int64_t)p * a.n_qblocks + qb) * a.splits + sp) * C::ROWS + rl) * (D + 4);
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4_t*>(pr + 32 * n + 8 * q + 4 * hf) =
            float4_t{acc[n][4 * q], acc[n][4 * q + 1], acc[n][4 * q + 2], acc[n][4 * q + 3]};
    }
    if (hf == 0) {
      pr[D] = m_ref;
      pr[D + 1] = l_tot;
    }
    return;
  }

  // ---- normalize and write this lane's half of row j ----
  if (DENSE ? row_live : pos < a.max_queries) {
    const float inv = (row_live && l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
    _Float16* op = DENSE ? a.out + (int64_t)(q0 + pos) * a.o_stride_t + (int64_t)head * a.o_stride_h
                         : a.out + (((int64_t)b * a.num_q_heads + head) * a.max_queries + pos) * D;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        half4_t o;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) o[rr] = (_Float16)(acc[n][4 * q + rr] * inv);
        *reinterpret_cast<half4_t*>(op + 32 * n + 8 * q + 4 * hf) = o;
      }
    }
  }
}

// The wide kernel serves the paged head_dim-128 calls whose tensors fit
// 32-bit offsets (no per-tile descriptor rebasing), with or without a window.
// Query rows per workgroup at this head_dim and layout (Cfg<D, K8V3>::ROWS,
// or WideCfg::ROWS for the wide kernel), and the workgroups a CU keeps
// resident (the kernels' launch bounds).
static bool use_wide(int head_dim, bool big) { return head_dim == 128 && !big; }
// rows: query rows per (sequence, KV head) -- group x max_queries; the wide
// kernel takes 8-wave workgroups when they exceed one 4-wave block
static bool wide_eight(int rows) { return rows > WideCfg<false, false>::ROWS; }
static int rows_per_wg(int head_dim, bool k8v3, bool wide, int rows) {
  if (wide) return wide_eight(rows) ? WideCfg<false, true>::ROWS : WideCfg<false, false>::ROWS;
  return 16 * (k8v3 ? 8 : 4) * (head_dim <= 64 ? 2 : 1);
}
static int wg_per_cu(bool k8v3, bool wide, int rows) {
  return wide ? (wide_eight(rows) ? WideCfg<false, true>::WG_PER_CU : WideCfg<false, false>::WG_PER_CU)
              : (k8v3 ? 1 : 2);
}

// Combine of a split verify: one thread per (row, 4 dims) of a (sequence,
// KV head, query block) merges the row's `splits` partials -- each relative to
// its own running max, so weighted by 2^(m_s - max m) -- and writes the
// normalized fp16 dims.  Workgroup x covers items kCombineThreads * (x %
// blocks_per_unit) .. of unit x / blocks_per_unit.
constexpr int kCombineThreads = 64;  // one wave: a batch-1 combine spreads over every CU
template <int D, int ROWS>
__global__ __launch_bounds__(kCombineThreads) void verify_combine_kernel(VerifyArgs a) {
  constexpr int V4 = D / 4;
  constexpr int BLOCKS = ROWS * V4 / kCombineThreads;  // workgroups per unit
  static_assert(ROWS * V4 % kCombineThreads == 0, "whole workgroups per unit");
  const int pq = blockIdx.x / BLOCKS;  // (sequence, KV head) * n_qblocks + query block
  const int it = (blockIdx.x - pq * BLOCKS) * kCombineThreads + threadIdx.x;
  const int p = pq / a.n_qblocks;
  const int qb = pq - p * a.n_qblocks;
  const int b = p / a.num_kv_heads;
  const int h = p - b * a.num_kv_heads;
  const int G = a.group;
  const int rl = it / V4;
  const int c4 = it - rl * V4;
  const int r = qb * ROWS + rl;
  const int pos = r / G;
  if (pos >= a.max_queries) return;
  const int head = h * G + (r - pos * G);
  half4_t* const op = reinterpret_cast<half4_t*>(a.out + (((int64_t)b * a.num_q_heads + head) * a.max_queries + pos) * D +
                                                 4 * c4);
  // rows past the sequence's query count are zeros, as the unsplit kernel writes them
  const int nq = a.query_lens ? max(0, min(a.query_lens[b], a.max_queries)) : a.max_queries;
  if (pos >= nq) {
    *op = half4_t{0, 0, 0, 0};
    return;
  }
  const int S = a.splits;
  const int64_t stride = (int64_t)ROWS * (D + 4);  // between splits of one row
  const float* row = a.part + ((int64_t)pq * S * ROWS + rl) * (D + 4);
  // one pass, 32 partials in flight: the running max rises batch by batch and
  // rescales what is summed so far (a split count of 64 reads in 2 rounds)
  constexpr int U = 32;
  float M = -__builtin_inff();
  float4_t num = float4_t{0.f, 0.f, 0.f, 0.f};
  float den = 0.0f;
  for (int s0 = 0; s0 < S; s0 += U) {
    float m[U], l[U];
    float4_t x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = min(s0 + u, S - 1);
      const float* pr = row + s * stride;
      m[u] = pr[D];
      l[u] = pr[D + 1];
      x[u] = *reinterpret_cast<const float4_t*>(pr + 4 * c4);
    }
    float mb = M;  // (partial maxima are finite: a split without keys keeps its initial max)
#pragma unroll
    for (int u = 0; u < U; ++u) mb = s0 + u < S ? fmaxf(mb, m[u]) : mb;
    const float c = __builtin_amdgcn_exp2f(M - mb);  // 0 on the first batch
    num *= c;
    den *= c;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float f = s0 + u < S ? __builtin_amdgcn_exp2f(m[u] - mb) : 0.0f;
      num += f * x[u];
      den += f * l[u];
    }
    M = mb;
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  half4_t o;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) o[rr] = (_Float16)(num[rr] * inv);
  *op = o;
}

// The combine of a split call: one single-wave workgroup per 64 (row, 4 dims)
// items of every unit.
template <int D, int ROWS>
static int launch_combine(VerifyArgs& a, int64_t units, hipStream_t stream) {
  const int64_t grid = units * (ROWS * (D / 4) / kCombineThreads);
  if (grid > INT32_MAX) {
    set_error("s8kv_verify: combine grid too large");
    return S8KV_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((verify_combine_kernel<D, ROWS>), dim3((unsigned)grid), dim3(kCombineThreads), 0, stream, a);
  return check_launch("s8kv_verify_combine");
}

template <int D, bool K8V3, bool WIN, bool DENSE, bool BIG>
static int launch_impl(VerifyArgs& a, hipStream_t stream) {
  static_assert(Cfg<D, K8V3>::ROWS == 16 * kWavesOf<K8V3> * (D <= 64 ? 2 : 1), "rows_per_wg");
  using C = Cfg<D, K8V3>;
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&verify_kernel<D, K8V3, WIN, DENSE, BIG>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, WIN ? C::SMEM_WIN : C::SMEM) != hipSuccess) {
      set_error("s8kv_verify: cannot set the dynamic LDS size");
      return S8KV_ERR_LAUNCH;
    }
    attr = true;
  }
  const int P = a.batch * a.num_kv_heads;
  const int64_t grid = (int64_t)8 * a.n_qblocks * a.splits * ((P + 7) / 8);
  if (grid > INT32_MAX) {
    set_error("s8kv_verify: grid too large");
    return S8KV_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((verify_kernel<D, K8V3, WIN, DENSE, BIG>), dim3((unsigned)grid), dim3(C::THREADS),
                     WIN ? C::SMEM_WIN : C::SMEM, stream, a);
  if (a.splits > 1) {
    const int rc = check_launch("s8kv_verify");
    if (rc != S8KV_OK) return rc;
    return launch_combine<D, C::ROWS>(a, (int64_t)P * a.n_qblocks, stream);
  }
  return check_launch("s8kv_verify");
}
template <int D, bool K8V3, bool WIN = false, bool DENSE = false>
static int launch(VerifyArgs& a, hipStream_t stream) {
  if constexpr (DENSE)
    return launch_impl<D, K8V3, WIN, DENSE, false>(a, stream);
  else
    return a.big ? launch_impl<D, K8V3, WIN, DENSE, true>(a, stream)
                 : launch_impl<D, K8V3, WIN, DENSE, false>(a, stream);
}

template <bool K8V3, bool DENSE, bool WIN, bool FRESH, bool EIGHT>
static int launch_wide_impl(VerifyArgs& a, hipStream_t stream) {
  using C = WideCfg<K8V3, EIGHT>;
  constexpr int smem = FRESH ? C::SMEM_WIN : C::SMEM;
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&verify_wide_kernel<K8V3, DENSE, WIN, FRESH, EIGHT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, smem) != hipSuccess) {
      set_error("s8kv_verify: cannot set the dynamic LDS size");
      return S8KV_ERR_LAUNCH;
    }
    attr = true;
  }
  const int P = a.batch * a.num_kv_heads;
  const int64_t grid = (int64_t)8 * a.n_qblocks * a.splits * ((P + 7) / 8);
  if (grid > INT32_MAX) {
    set_error("s8kv_verify: grid too large");
    return S8KV_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((verify_wide_kernel<K8V3, DENSE, WIN, FRESH, EIGHT>), dim3((unsigned)grid), dim3(C::THREADS), smem,
                     stream, a);
  if (a.splits > 1) {
    const int rc = check_launch("s8kv_verify");
    if (rc != S8KV_OK) return rc;
    return launch_combine<C::D, C::ROWS>(a, (int64_t)P * a.n_qblocks, stream);
  }
  return check_launch("s8kv_verify");
}

// 8-wave workgroups for calls with more than 128 query rows per (sequence,
// KV head) (a batch-1 32-node tree at G 4 would leave half of their waves
// idle: 13 % slower); the host sized n_qblocks and the split by the same
// rule (rows_per_wg, wg_per_cu)
template <bool K8V3, bool DENSE = false, bool WIN = false, bool FRESH = false>
static int launch_wide(VerifyArgs& a, hipStream_t stream) {
  if (wide_eight(a.group * a.max_queries)) return launch_wide_impl<K8V3, DENSE, WIN, FRESH, true>(a, stream);
  return launch_wide_impl<K8V3, DENSE, WIN, FRESH, false>(a, stream);
}

}  // namespace verify
}  // namespace s8kv

using namespace s8kv;

// Optional fresh fp16 drafts of the window verify: K (rotated) and V, element
// strides per row, draft and head.
struct FreshDrafts {
  const void* k;
  const void* v;
  int64_t k_stride[3];
  int64_t v_stride[3];
};

// Key-range split of the paged verify.  A launch with fewer workgroups than
// the GPU keeps resident (two per CU) leaves CUs idle for the whole call --
// batch-1 speculative decoding with a long context is the common case -- so
// each (sequence, KV head, query block) is split until about that many
// exist, down to kMinSplitKeys keys per split (512: a 32K-key batch-1 tree
// verify at 8 KV heads fills all 512 slots, 4-5 % faster than 32 splits of
// 1024 keys; a second round of splits is slower again); and one workgroup
// never accumulates more than kMaxSplitKeys keys, which bounds the rounding
// of its fp32 sums.  s8kv_verify_set_splits overrides the count (diagnostics).
constexpr int kMinSplitKeys = 512;
constexpr int kMaxSplitKeys = 1 << 20;
constexpr int kMaxSplits = 1024;
static std::atomic<int> g_verify_splits{0};  // 0: planned per call
static int verify_plan_splits(int batch, int num_kv_heads, int n_qblocks, int keys, bool k8v3, bool wide, int rows) {
  const int64_t natural = (int64_t)batch * num_kv_heads * n_qblocks;
  const int64_t resident = (int64_t)verify::wg_per_cu(k8v3, wide, rows) * device_cus();
  int64_t s = natural < resident ? (resident + natural - 1) / natural : 1;
  s = std::min<int64_t>(s, std::max(1, keys / kMinSplitKeys));
  s = std::max<int64_t>(s, ((int64_t)keys + kMaxSplitKeys - 1) / kMaxSplitKeys);
  const int forced = g_verify_splits.load();
  if (forced > 0) s = forced;
  return (int)std::max<int64_t>(1, std::min<int64_t>(s, kMaxSplits));
}
static int64_t verify_part_bytes(int batch, int num_kv_heads, int n_qblocks, int head_dim, int splits, bool k8v3,
                                 bool wide, int rows) {
  if (splits <= 1) return 0;
  return (int64_t)batch * num_kv_heads * n_qblocks * splits * verify::rows_per_wg(head_dim, k8v3, wide, rows) *
         (head_dim + 4) * 4;
}

extern "C" int64_t s8kv_verify_workspace_size(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                              int max_queries, int max_context_len) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || max_queries <= 0 ||
      max_context_len < 0 || (head_dim != 64 && head_dim != 128 && head_dim != 256))
    return 0;
  // either layout and kernel (their workgroups differ in query rows): the larger need
  int64_t need = 0;
  for (const bool k8v3 : {false, true}) {
    for (const bool wide : {false, true}) {
      if (wide && head_dim != 128) continue;
      const int rows = num_q_heads / num_kv_heads * max_queries;
      const int rows_wg = verify::rows_per_wg(head_dim, k8v3, wide, rows);
      const int n_qblocks = (rows + rows_wg - 1) / rows_wg;
      need = std::max(need, verify_part_bytes(batch, num_kv_heads, n_qblocks, head_dim,
                                              verify_plan_splits(batch, num_kv_heads, n_qblocks, max_context_len,
                                                                 k8v3, wide, rows),
                                              k8v3, wide, rows));
    }
  }
  return need;
}

// The split for this call (keys: the most any block reads -- a window layer's
// window and drafts), used when the caller's workspace holds its partials;
// never more than s8kv_verify_workspace_size plans for, which counts
// max_context_len keys.  A split made only to fill the GPU is dropped when
// the workspace cannot hold it (the call is then slower, not different in
// kind); a block reading more than kMaxSplitKeys keys must split, so then a
// missing or short workspace is an error.
static int verify_use_workspace(verify::VerifyArgs& a, int head_dim, bool k8v3, bool wide, void* workspace,
                                int64_t workspace_bytes) {
  const int keys = a.window > 0 ? (int)std::min<int64_t>(a.max_context_len, (int64_t)a.window + a.max_queries)
                                : a.max_context_len;
  const int rows = a.group * a.max_queries;
  const int s = verify_plan_splits(a.batch, a.num_kv_heads, a.n_qblocks, keys, k8v3, wide, rows);
  const int64_t need = verify_part_bytes(a.batch, a.num_kv_heads, a.n_qblocks, head_dim, s, k8v3, wide, rows);
  const bool fits = workspace != nullptr && workspace_bytes >= need && (uintptr_t)workspace % 16 == 0;
  if (s > 1 && fits) {
    a.splits = s;
    a.part = (float*)workspace;
  }
  S8KV_REQUIRE(fits || keys <= kMaxSplitKeys, S8KV_ERR_WORKSPACE,
               "verify: %d keys per block exceed %d without a split: a 16-byte aligned workspace of %lld bytes "
               "(s8kv_verify_workspace_size) is needed, %lld given", keys, kMaxSplitKeys, (long long)need,
               (long long)(workspace ? workspace_bytes : 0));
  return S8KV_OK;
}

extern "C" int s8kv_verify_set_splits(int splits) {
  S8KV_REQUIRE(splits >= 0 && splits <= kMaxSplits, S8KV_ERR_INVALID, "verify_set_splits: %d not in [0, %d]", splits,
               kMaxSplits);
  g_verify_splits.store(splits);
  return S8KV_OK;
}

// Checks and arguments shared by both layouts (everything but V).
static int verify_setup(verify::VerifyArgs& a, const void* q, int batch, int num_q_heads, int num_kv_heads,
                        int head_dim, int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                        const int8_t* k_cache, const float* k_scale, int64_t num_blocks, int block_size,
                        const int32_t* block_table, int64_t block_table_stride, const int32_t* prefix_lens,
                        const int32_t* query_lens, const int64_t* tree_mask, int max_context_len, float scale,
                        void* out, bool k8v3) {
  S8KV_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0, S8KV_ERR_INVALID,
               "verify: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads, num_kv_heads);
  S8KV_REQUIRE(num_q_heads / num_kv_heads <= 16, S8KV_ERR_UNSUPPORTED, "verify: more than 16 q heads per kv head");
  S8KV_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, S8KV_ERR_UNSUPPORTED,
               "verify: head_dim %d not in {64, 128, 256}", head_dim);
  S8KV_REQUIRE(is_pow2(block_size) && block_size >= 4, S8KV_ERR_UNSUPPORTED,
               "verify: block_size %d must be a power of two >= 4", block_size);
  S8KV_REQUIRE(num_blocks > 0 && max_context_len >= 0, S8KV_ERR_INVALID, "verify: bad num_blocks/max_context_len");
  S8KV_REQUIRE(q && k_cache && k_scale && block_table && prefix_lens && out, S8KV_ERR_INVALID,
               "verify: null pointer argument");
  const int64_t rows = num_blocks * num_kv_heads * block_size;
  S8KV_REQUIRE(fits_u32(rows), S8KV_ERR_UNSUPPORTED, "verify: more than 2^32 cache rows per layer");
  // a tensor past 4 GiB: tiles through descriptors rebased per tile, which
  // needs tiles inside one block
  a.big = !fits_u32(rows * head_dim);
  S8KV_REQUIRE(!a.big || block_size >= 32, S8KV_ERR_UNSUPPORTED,
               "verify: a per-layer cache past 4 GiB needs block_size >= 32 (got %d)", block_size);
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.q_stride_s = q_stride_s;
  a.batch = batch;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.max_queries = max_queries;
  a.k_cache = k_cache;
  a.k_scale = k_scale;
  a.kc_total = (uint64_t)(rows * head_dim);
  a.ks_total = (uint64_t)(rows * 4);
  a.kc_bytes = cap_u32(a.kc_total);  // (BIG: unused by the tiles)
  a.ks_bytes = cap_u32(a.ks_total);
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.prefix_lens = prefix_lens;
  a.query_lens = query_lens;
  a.tree_mask = tree_mask;
  a.bs_log2 = log2i(block_size);
  a.max_context_len = max_context_len;
  const int rows_wg = verify::rows_per_wg(head_dim, k8v3, verify::use_wide(head_dim, a.big), a.group * max_queries);
  a.n_qblocks = (a.group * max_queries + rows_wg - 1) / rows_wg;
  a.qscale = (float)((double)scale * 1.4426950408889634 / __builtin_sqrt((double)head_dim));
  a.out = (_Float16*)out;
  return S8KV_OK;
}

static int verify_int8_impl(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                                const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                                const float* v_scale, int64_t num_blocks, int block_size, const int32_t* block_table,
                                int64_t block_table_stride, const int32_t* prefix_lens, const int32_t* query_lens,
                                const int64_t* tree_mask, int max_context_len, float scale, void* out,
                                void* workspace, int64_t workspace_bytes, void* stream, int window,
                                const FreshDrafts* fresh) {
  S8KV_REQUIRE(batch >= 0 && max_queries >= 0, S8KV_ERR_INVALID, "verify: negative batch or query count");
  if (batch == 0 || max_queries == 0) return S8KV_OK;
  const bool fresh_k = fresh != nullptr && fresh->k != nullptr;
  verify::VerifyArgs a{};
  a.splits = 1;
  const int rc = verify_setup(a, q, batch, num_q_heads, num_kv_heads, head_dim, max_queries, q_stride_b, q_stride_h,
                              q_stride_s, k_cache, k_scale, num_blocks, block_size, block_table, block_table_stride,
                              prefix_lens, query_lens, tree_mask, max_context_len, scale, out, false);
  if (rc != S8KV_OK) return rc;
  a.window = window;
  const bool wide = verify::use_wide(head_dim, a.big);
  if (const int rc = verify_use_workspace(a, head_dim, false, wide, workspace, workspace_bytes)) return rc;
  if (fresh_k) {
    S8KV_REQUIRE(fresh->v != nullptr && window > 0, S8KV_ERR_INVALID, "verify: fresh drafts need V and a window");
    S8KV_REQUIRE((uintptr_t)fresh->k % 16 == 0 && (uintptr_t)fresh->v % 16 == 0 && fresh->k_stride[0] % 4 == 0 &&
                     fresh->k_stride[1] % 4 == 0 && fresh->k_stride[2] % 4 == 0 && fresh->v_stride[0] % 8 == 0 &&
                     fresh->v_stride[1] % 8 == 0 && fresh->v_stride[2] % 8 == 0,
                 S8KV_ERR_INVALID, "verify: fresh draft rows must be 16-byte aligned");
    a.kd = (const float*)fresh->k;
    a.vd = (const _Float16*)fresh->v;
    a.kd_stride_b = fresh->k_stride[0];
    a.kd_stride_s = fresh->k_stride[1];
    a.kd_stride_h = fresh->k_stride[2];
    a.vd_stride_b = fresh->v_stride[0];
    a.vd_stride_s = fresh->v_stride[1];
    a.vd_stride_h = fresh->v_stride[2];
  }
  S8KV_REQUIRE(v_cache && v_scale, S8KV_ERR_INVALID, "verify: null pointer argument");
  a.v_cache = v_cache;
  a.v_scale = v_scale;
  a.vc_total = a.kc_total;
  a.vs_total = a.ks_total;
  a.vc_bytes = a.kc_bytes;
  a.vs_bytes = a.ks_bytes;
  hipStream_t s = (hipStream_t)stream;
  if (wide) {
    if (a.kd != nullptr) return verify::launch_wide<false, false, true, true>(a, s);
    return a.window > 0 ? verify::launch_wide<false, false, true>(a, s) : verify::launch_wide<false>(a, s);
  }
  if (a.window > 0) {
    switch (head_dim) {
      case 64: return verify::launch<64, false, true>(a, s);
      case 128: return verify::launch<128, false, true>(a, s);
      case 256: return verify::launch<256, false, true>(a, s);
    }
    return S8KV_ERR_UNSUPPORTED;
  }
  switch (head_dim) {
    case 64: return verify::launch<64, false>(a, s);
    case 128: return verify::launch<128, false>(a, s);
    case 256: return verify::launch<256, false>(a, s);
  }
  return S8KV_ERR_UNSUPPORTED;
}

extern "C" int s8kv_verify_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                                const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                                const float* v_scale, int64_t num_blocks, int block_size, const int32_t* block_table,
                                int64_t block_table_stride, const int32_t* prefix_lens, const int32_t* query_lens,
                                const int64_t* tree_mask, int max_context_len, float scale, void* out,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  return verify_int8_impl(q, batch, num_q_heads, num_kv_heads, head_dim, max_queries, q_stride_b, q_stride_h,
                          q_stride_s, k_cache, k_scale, v_cache, v_scale, num_blocks, block_size, block_table,
                          block_table_stride, prefix_lens, query_lens, tree_mask, max_context_len, scale, out,
                          workspace, workspace_bytes, stream, 0, nullptr);
}

extern "C" int s8kv_verify_window_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                                const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                                const float* v_scale, int64_t num_blocks, int block_size, const int32_t* block_table,
                                int64_t block_table_stride, const int32_t* prefix_lens, const int32_t* query_lens,
                                const int64_t* tree_mask, int max_context_len, int window, const void* k_draft,
                                int64_t kd_stride_b, int64_t kd_stride_s, int64_t kd_stride_h, const void* v_draft,
                                int64_t vd_stride_b, int64_t vd_stride_s, int64_t vd_stride_h, float scale, void* out,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  S8KV_REQUIRE(window >= 1, S8KV_ERR_INVALID, "verify_window: window %d < 1", window);
  const FreshDrafts fresh{k_draft, v_draft, {kd_stride_b, kd_stride_s, kd_stride_h},
                          {vd_stride_b, vd_stride_s, vd_stride_h}};
  return verify_int8_impl(q, batch, num_q_heads, num_kv_heads, head_dim, max_queries, q_stride_b, q_stride_h,
                          q_stride_s, k_cache, k_scale, v_cache, v_scale, num_blocks, block_size, block_table,
                          block_table_stride, prefix_lens, query_lens, tree_mask, max_context_len, scale, out,
                          workspace, workspace_bytes, stream, window, &fresh);
}


static int verify_k8v3_impl(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                                const int8_t* k_cache, const float* k_scale, const int32_t* v_packed,
                                const float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                                int block_size, const int32_t* block_table, int64_t block_table_stride,
                                const int32_t* prefix_lens, const int32_t* query_lens, const int64_t* tree_mask,
                                int max_context_len, float scale, void* out, void* workspace,
                                int64_t workspace_bytes, void* stream, int window, const FreshDrafts* fresh) {
  S8KV_REQUIRE(batch >= 0 && max_queries >= 0, S8KV_ERR_INVALID, "verify: negative batch or query count");
  if (batch == 0 || max_queries == 0) return S8KV_OK;
  S8KV_REQUIRE(head_dim == 128 || head_dim == 256, S8KV_ERR_UNSUPPORTED,
               "verify k8v3: head_dim %d not in {128, 256}", head_dim);
  S8KV_REQUIRE(lloyd_block == 128, S8KV_ERR_UNSUPPORTED, "verify k8v3: lloyd_block %d != 128", lloyd_block);
  const bool fresh_k = fresh != nullptr && fresh->k != nullptr;
  verify::VerifyArgs a{};
  a.splits = 1;
  const int rc = verify_setup(a, q, batch, num_q_heads, num_kv_heads, head_dim, max_queries, q_stride_b, q_stride_h,
                              q_stride_s, k_cache, k_scale, num_blocks, block_size, block_table, block_table_stride,
                              prefix_lens, query_lens, tree_mask, max_context_len, scale, out, true);
  if (rc != S8KV_OK) return rc;
  a.window = window;
  const bool wide = verify::use_wide(head_dim, a.big);
  if (const int rc = verify_use_workspace(a, head_dim, true, wide, workspace, workspace_bytes)) return rc;
  if (fresh_k) {
    S8KV_REQUIRE(fresh->v != nullptr && window > 0, S8KV_ERR_INVALID, "verify: fresh drafts need V and a window");
    S8KV_REQUIRE((uintptr_t)fresh->k % 16 == 0 && (uintptr_t)fresh->v % 16 == 0 && fresh->k_stride[0] % 4 == 0 &&
                     fresh->k_stride[1] % 4 == 0 && fresh->k_stride[2] % 4 == 0 && fresh->v_stride[0] % 8 == 0 &&
                     fresh->v_stride[1] % 8 == 0 && fresh->v_stride[2] % 8 == 0,
                 S8KV_ERR_INVALID, "verify: fresh draft rows must be 16-byte aligned");
    a.kd = (const float*)fresh->k;
    a.vd = (const _Float16*)fresh->v;
    a.kd_stride_b = fresh->k_stride[0];
    a.kd_stride_s = fresh->k_stride[1];
    a.kd_stride_h = fresh->k_stride[2];
    a.vd_stride_b = fresh->v_stride[0];
    a.vd_stride_s = fresh->v_stride[1];
    a.vd_stride_h = fresh->v_stride[2];
  }
  S8KV_REQUIRE(v_packed && v_norm && v_codebook, S8KV_ERR_INVALID, "verify: null pointer argument");
  const int64_t rows = num_blocks * num_kv_heads * block_size;
  a.v_cache = v_packed;
  a.v_scale = v_norm;
  a.v_codebook = v_codebook;
  a.vc_total = (uint64_t)(rows * (head_dim / 32 * 3) * 4);
  a.vs_total = (uint64_t)(rows * (head_dim / 128) * 4);
  a.vc_bytes = cap_u32(a.vc_total);
  a.vs_bytes = cap_u32(a.vs_total);
  hipStream_t s = (hipStream_t)stream;
  if (wide) {
    if (a.kd != nullptr) return verify::launch_wide<true, false, true, true>(a, s);
    return a.window > 0 ? verify::launch_wide<true, false, true>(a, s) : verify::launch_wide<true>(a, s);
  }
  if (a.window > 0)
    return head_dim == 128 ? verify::launch<128, true, true>(a, s) : verify::launch<256, true, true>(a, s);
  return head_dim == 128 ? verify::launch<128, true>(a, s) : verify::launch<256, true>(a, s);
}

extern "C" int s8kv_verify_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                                const int8_t* k_cache, const float* k_scale, const int32_t* v_packed,
                                const float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                                int block_size, const int32_t* block_table, int64_t block_table_stride,
                                const int32_t* prefix_lens, const int32_t* query_lens, const int64_t* tree_mask,
                                int max_context_len, float scale, void* out, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  return verify_k8v3_impl(q, batch, num_q_heads, num_kv_heads, head_dim, max_queries, q_stride_b, q_stride_h,
                          q_stride_s, k_cache, k_scale, v_packed, v_norm, v_codebook, lloyd_block, num_blocks,
                          block_size, block_table, block_table_stride, prefix_lens, query_lens, tree_mask,
                          max_context_len, scale, out, workspace, workspace_bytes, stream, 0, nullptr);
}

extern "C" int s8kv_verify_window_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int max_queries, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
                                const int8_t* k_cache, const float* k_scale, const int32_t* v_packed,
                                const float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                                int block_size, const int32_t* block_table, int64_t block_table_stride,
                                const int32_t* prefix_lens, const int32_t* query_lens, const int64_t* tree_mask,
                                int max_context_len, int window, const void* k_draft, int64_t kd_stride_b,
                                int64_t kd_stride_s, int64_t kd_stride_h, const void* v_draft, int64_t vd_stride_b,
                                int64_t vd_stride_s, int64_t vd_stride_h, float scale, void* out, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  S8KV_REQUIRE(window >= 1, S8KV_ERR_INVALID, "verify_window: window %d < 1", window);
  const FreshDrafts fresh{k_draft, v_draft, {kd_stride_b, kd_stride_s, kd_stride_h},
                          {vd_stride_b, vd_stride_s, vd_stride_h}};
  return verify_k8v3_impl(q, batch, num_q_heads, num_kv_heads, head_dim, max_queries, q_stride_b, q_stride_h,
                          q_stride_s, k_cache, k_scale, v_packed, v_norm, v_codebook, lloyd_block, num_blocks,
                          block_size, block_table, block_table_stride, prefix_lens, query_lens, tree_mask,
                          max_context_len, scale, out, workspace, workspace_bytes, stream, window, &fresh);
}


extern "C" int s8kv_attn_varlen_f16(const void* q, const void* k, const void* v, const int32_t* cu_seqlens_q,
                                    const int32_t* cu_seqlens_k, int batch, int num_q_heads, int num_kv_heads,
                                    int head_dim, int max_seqlen_q, int max_seqlen_k, int64_t q_stride_t,
                                    int64_t q_stride_h, int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t,
                                    int64_t v_stride_h, int causal, int window_left, float scale, void* out,
                                    int64_t o_stride_t, int64_t o_stride_h, void* stream) {
  S8KV_REQUIRE(batch >= 0 && max_seqlen_q >= 0 && max_seqlen_k >= 0, S8KV_ERR_INVALID,
               "attn_varlen: negative batch or sequence length");
  if (batch == 0 || max_seqlen_q == 0) return S8KV_OK;
  S8KV_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0, S8KV_ERR_INVALID,
               "attn_varlen: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads, num_kv_heads);
  S8KV_REQUIRE(num_q_heads / num_kv_heads <= 16, S8KV_ERR_UNSUPPORTED, "attn_varlen: more than 16 q heads per kv head");
  S8KV_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, S8KV_ERR_UNSUPPORTED,
               "attn_varlen: head_dim %d not in {64, 128, 256}", head_dim);
  S8KV_REQUIRE(q && k && v && cu_seqlens_q && cu_seqlens_k && out, S8KV_ERR_INVALID,
               "attn_varlen: null pointer argument");
  S8KV_REQUIRE(window_left < 0 || causal, S8KV_ERR_UNSUPPORTED, "attn_varlen: window_left needs causal");
  S8KV_REQUIRE(window_left != 0, S8KV_ERR_INVALID, "attn_varlen: window_left 0 would leave no key (>= 1, or -1)");
  S8KV_REQUIRE((uintptr_t)k % 16 == 0 && (uintptr_t)v % 16 == 0 && k_stride_t % 8 == 0 && k_stride_h % 8 == 0 &&
                   v_stride_t % 8 == 0 && v_stride_h % 8 == 0,
               S8KV_ERR_INVALID, "attn_varlen: K and V rows must be 16-byte aligned");
  verify::VerifyArgs a{};
  a.splits = 1;
  a.q = (const _Float16*)q;
  a.q_stride_s = q_stride_t;
  a.q_stride_h = q_stride_h;
  a.batch = batch;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.max_queries = max_seqlen_q;
  a.max_context_len = max_seqlen_k;
  a.bs_log2 = 5;
  const int rows_wg = verify::rows_per_wg(head_dim, false, false, 0);
  a.n_qblocks = (a.group * max_seqlen_q + rows_wg - 1) / rows_wg;
  a.qscale = (float)((double)scale * 1.4426950408889634);  // K is not rotated: no 1/sqrt(D)
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.k_f16 = (const _Float16*)k;
  a.v_f16 = (const _Float16*)v;
  a.k_stride_t = k_stride_t;
  a.k_stride_h = k_stride_h;
  a.v_stride_t = v_stride_t;
  a.v_stride_h = v_stride_h;
  a.o_stride_t = o_stride_t;
  a.o_stride_h = o_stride_h;
  a.causal = causal ? 1 : 0;
  a.out = (_Float16*)out;
  hipStream_t s = (hipStream_t)stream;
  // head_dim 128: the wide kernel (32 query rows per wave) when its vector
  // q loads (16 bytes) and output stores (8 bytes) are aligned
  const bool wide = head_dim == 128 && (uintptr_t)q % 16 == 0 && q_stride_t % 8 == 0 && q_stride_h % 8 == 0 &&
                    (uintptr_t)out % 8 == 0 && o_stride_t % 4 == 0 && o_stride_h % 4 == 0;
  if (wide)
    a.n_qblocks = (a.group * max_seqlen_q + verify::rows_per_wg(128, false, true, a.group * max_seqlen_q) - 1) /
                  verify::rows_per_wg(128, false, true, a.group * max_seqlen_q);
  if (window_left > 0) {  // query s sees keys (s + nk - nq - window_left, s + nk - nq]: window_left keys
    a.window = window_left - 1;  // the kernel's band: keys >= s + nk - nq - window
    if (wide) return verify::launch_wide<false, true, true>(a, s);
    switch (head_dim) {
      case 64: return verify::launch<64, false, true, true>(a, s);
      case 128: return verify::launch<128, false, true, true>(a, s);
      case 256: return verify::launch<256, false, true, true>(a, s);
    }
    return S8KV_ERR_UNSUPPORTED;
  }
  if (wide) return verify::launch_wide<false, true>(a, s);
  switch (head_dim) {
    case 64: return verify::launch<64, false, false, true>(a, s);
    case 128: return verify::launch<128, false, false, true>(a, s);
    case 256: return verify::launch<256, false, false, true>(a, s);
  }
  return S8KV_ERR_UNSUPPORTED;
}
