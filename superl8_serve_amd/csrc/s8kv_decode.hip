// Ragged-batch GQA decode attention over the paged int8 / K8V3 cache.
//
// Scheduling (stream-K): the grid holds about as many workgroups as the GPU
// keeps resident, wg_per_head of them per KV head.  For its head, each
// workgroup takes an equal, contiguous slice of the concatenation of all rows'
// tokens (each row padded to a multiple of 32), so ragged context lengths
// never leave part of the GPU idle.  A slice may end inside one row and start
// the next; the part of a row inside one slice is a "segment".  A row covered
// by a single segment is written directly, otherwise every segment writes a
// (max, sum, acc) partial and the workgroup whose segment completes the row
// (see "Arrival counters" below) combines them.  Each row also
// occupies `ghost` stream tokens that are not processed: they charge the fixed
// cost of a segment (q set-up, merge) to the slice that holds it.  A
// segment's set-up loads (q, first block ids) are issued before the previous
// segment's merge so their latency hides behind it.  Workgroup id
// wg = j * Hkv + h: the round-robin deal of workgroups to the 8 XCDs gives
// every XCD the same number of equal-work workgroups (with Hkv = 8, all of
// head h's on XCD h, whose L2 then holds that head's block table and q).
//
// Inside a segment the 4 waves of the workgroup take 32-token tiles in turn
// (tiles w, w+4, ...) and keep an online softmax for the G = Hq/Hkv query heads
// of the KV head, so every KV byte is read once for all G heads.  Per tile:
//   QK  : S[token][head] on MFMA 16x16x32 f16.  A = K rows (int8 -> fp16 is
//         exact) loaded straight from HBM in MFMA operand layout; B = the
//         rotated, pre-scaled q split into fp16 hi + lo parts (two MFMAs), so
//         scores carry ~22 bits of q precision.
//   softmax: lane (head c = lane%16, group g = lane/16) owns tokens
//         {4g..4g+3} and {16+4g..16+4g+3} of the tile; the running max is
//         shared across the 4 groups with two lane shuffles.
//   PV  : O^T[dim][head] on MFMA 16x16x32 f16.  B = P^T from the lane's own
//         softmax values (times the per-token V scale / norm, split into fp16
//         hi + lo) -- no shuffle; A = V^T read from an LDS copy of the tile
//         with the gfx950 transpose reads ds_read_b64_tr_b8 (int8) /
//         ds_read_b64_tr_b16 (K8V3 codes expanded to fp16 in LDS).
// The next tile's loads are issued while the current one computes.
//
// Arrival counters: the partials of a split row are stored with agent-scope
// (L2-bypassing, `sc1`) stores; after every wave has waited for its stores,
// one lane adds the segment's length to the row's counter word with an
// agent-scope compare-and-swap, and the workgroup that brings the count to the
// row's padded length reads the partials back with agent-scope loads and
// writes the row.  Only the data exchanged goes through the coherence point:
// agent-scope release/acquire fences would write back and invalidate the
// whole L2 of the XCD instead.  A counter word holds a 40-bit tag of the
// launch and a 24-bit count of 32-token units; a word whose tag is not this
// launch's counts as zero, so the workspace needs no initialisation (a stale
// word matches a launch's tag with probability 2^-40), and the last arrival
// writes the word back to zero, so a graph replaying the launch with the same
// tag starts from zero too.
#include <stdlib.h>
#include <unistd.h>

#include <atomic>
#include <chrono>

#include <array>
#include <mutex>
#include <type_traits>
#include <vector>

#include <hip/hip_ext.h>

#include "s8kv_device.h"
#include "s8kv_host.h"

namespace s8kv {

// Diagnostics build only (libsuperl8_kv_trace.so, compiled with
// -DS8KV_DECODE_TRACE): each workgroup stamps the device's constant 100 MHz
// clock at fixed points of its run and writes one 16-word record at its end
// (kTraceWords below); the product library compiles none of it.
#ifdef S8KV_DECODE_TRACE
enum TraceSlot {
  kTrEntry = 0,      // workgroup start
  kTrLens = 1,       // context lengths staged in LDS
  kTrFound = 2,      // slice and first segment located
  kTrStaged = 3,     // first segment's q and block ids loaded (block ids staged)
  kTrQ = 4,          // first segment's rotated q published
  kTrTile1 = 5,      // wave 0's first full tile done
  kTrTilesEnd = 6,   // wave 0 left the last segment's tile loop
  kTrExit = 7,       // workgroup end
  kTrWork = 8,       // tokens processed | segments << 32
  kTrFlags = 9,      // 1 | last segment whole row << 8 | last segment combined its row << 9
  kTrHwId = 10,      // the workgroup's XCC, shader engine and CU (__smid)
};
constexpr int kTraceWords = 16;
#define S8KV_TRACE_STAMP(slot)                                                 \
  do {                                                                         \
    if (threadIdx.x == 0) trace_lds[slot] = __builtin_amdgcn_s_memrealtime();  \
  } while (0)
#define S8KV_TRACE_STAMP_ONCE(slot)                                                          \
  do {                                                                                       \
    if (threadIdx.x == 0 && trace_lds[slot] == 0) trace_lds[slot] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define S8KV_TRACE_SET(slot, value)                 \
  do {                                              \
    if (threadIdx.x == 0) trace_lds[slot] = (value); \
  } while (0)
#else
#define S8KV_TRACE_STAMP(slot) \
  do {                         \
  } while (0)
#define S8KV_TRACE_STAMP_ONCE(slot) \
  do {                              \
  } while (0)
#define S8KV_TRACE_SET(slot, value) \
  do {                              \
  } while (0)
#endif

constexpr int kDecWaves = 4;
// Cache policy of the tile loads (K, V, scales): non-temporal for the int8
// layout, whose loads read whole lines once (a read-only sweep over the
// decode's tiles: 5.6 -> 6.3 TB/s); the default for K8V3, where
// non-temporal loads measured slower (4-13 % with each code group's words
// as three dword loads, 2 % with one dwordx3 load).
template <bool K8V3>
constexpr int kTilePolicy = K8V3 ? 0 : kNT;
constexpr int kTile = 32;
constexpr float kNegInf = -__builtin_inff();
constexpr float kMaxSlack = 8.0f;                        // lazy softmax max: rescale only past this (log2 units)
constexpr int kSubTokens = 2048;                         // block ids are staged in LDS per 2048 tokens
constexpr int kMaxSubBlocks = kSubTokens / 4 + 2;        // block_size >= 4
constexpr int kMaxResidentPerCU = 8;                     // bound used to size the workspace
constexpr int kLensLds = 1024;                           // context lengths kept in LDS (rows beyond: global reads)
constexpr int kGhostTokens = 192;                        // stream tokens charged per row start
constexpr int kSlotSkewPermille = 200;                   // slice weight skew across residency slots
constexpr int kQHeadsPerWave = 4;                        // q heads a wave rotates (group <= 16, 4 waves)

template <int D, bool K8V3>
struct DecCfg {
  static constexpr int KCH = D / 4;          // K bytes per lane per token row
  static constexpr int NQK = D / 32;         // QK MFMAs per 16-token subtile
  static constexpr int NPV = D / 16;         // PV MFMAs per tile (16 dims each)
  static constexpr int NB = K8V3 ? D / 128 : 1;  // per-token V scales: 1 (int8) or Lloyd-Max blocks (K8V3)
  static constexpr int NG = D / 32;          // 32-dim code groups per row (K8V3)
  static constexpr int WORDS = NG * 3;       // packed words per row (K8V3)
  // LDS row pitch of the staged V tile: int8 rows padded by 16 B, fp16 rows by
  // 32 B, so the 8 (int8) / 4 (fp16) rows one transpose read touches fall in
  // distinct banks.
  static constexpr int VROW = K8V3 ? (2 * D + 32) : (D + 16);
  static constexpr int VSTAGE = kTile * VROW;                 // bytes per wave
  static constexpr int VLOADS = K8V3 ? (kTile * NG) / 64 : (kTile * D / 16) / 64;  // V loads per lane per tile
  static constexpr int SMEM_A = kDecWaves * VSTAGE;
  static constexpr int SMEM_Q = (SMEM_A + 15) / 16 * 16;   // rotated q (hi, lo) [2][G][D] fp16, after the V staging
  // fused append: the new token's rows in LDS -- fp16 K and V (staged at the
  // segment start), int8 K, then int8 V (int8) or packed V words (K8V3), then
  // the K scale and the V scale (int8) or V norms (K8V3)
  static constexpr int NEW_F16K = 0, NEW_F16V = 2 * D, NEW_I8K = 4 * D, NEW_V = 5 * D;
  static constexpr int NEW_KS = K8V3 ? NEW_V + 4 * WORDS : NEW_V + D;
  static constexpr int NEW_VS = NEW_KS + 4;
  static constexpr int NEW_BYTES = (NEW_VS + 4 * NB + 15) / 16 * 16;
};

struct DecodeArgs {
  const _Float16* q;
  int64_t q_stride_b, q_stride_h;
  int batch, num_q_heads, num_kv_heads, group;
  const void* k_cache;
  const void* k_scale;
  const void* v_cache;   // int8 V or int32 packed V
  const void* v_scale;   // fp32 V scale or fp32 V norms
  const float* v_codebook;
  uint32_t kc_bytes, ks_bytes, vc_bytes, vs_bytes;
  // the tensors' full sizes; decode_kernel<.., BIG> (a tensor past 4 GiB,
  // block_size >= 32) addresses each tile through a descriptor rebased to it
  uint64_t kc_total, ks_total, vc_total, vs_total;
  int big;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* context_lens;
  int bs_log2;
  int max_context_len;  // every row is clamped to it (block-table rows hold this many tokens)
  int smem_main;        // LDS bytes before the staged block ids (V staging, then the merge)
  int wg_per_head;      // workgroups per KV head (slices of the token stream)
  int slots;            // partial slots per head: batch + wg_per_head
  int ghost;            // stream tokens charged per row for its fixed costs (multiple of 32)
  int slot_classes;     // residency slots per CU the grid fills (slice weighting classes)
  int slot_skew;        // slice weight skew between the first and last slot, in 1/1000
  float qscale;         // softmax scale * log2(e) * 1/sqrt(D) (rotation norm)
  _Float16* out;
  float* ws_ml;         // [Hkv][slots][G][2]  (max, sum) of each segment
  float* ws_acc;        // [Hkv][slots][G][D]  unnormalized output of each segment
  unsigned long long* ws_cnt;  // [Hkv][batch] arrival counters: tag << 24 | 32-token units done
  unsigned long long tag;      // this launch's 40-bit tag (non-zero)
  // fused append (decode_kernel<D, false, true>): row b's new token, at position
  // context_lens[b] - 1, is quantized and written by the workgroup that holds
  // the row's last tile, which attends over it from registers
  const _Float16* k_new;  // [batch][Hkv][D] fp16, unit stride on D
  const _Float16* v_new;
  int64_t kn_stride_b, kn_stride_h, vn_stride_b, vn_stride_h;
  float rot_norm;         // fp32(1/sqrt(D)): the K rotation's normalisation
  int smem_new;           // LDS byte offset of the new token's rows (DecCfg NEW_*)
  // sliding window (decode_kernel<D, K8V3, false, true>): row b attends only
  // its last `window` tokens (window >= 1)
  int window;
  // per-step slice plan (decode_plan_kernel; null: the prologue computes it)
  const int32_t* plan;
  int plan_wmax;      // workgroup columns the plan buffer's layout is sized for (max_wg_per_head)
  int32_t* plan_out;  // host only: s8kv_decode_plan writes the plan here instead of decoding
  int plan_adapt;     // host only: s8kv_decode_plan_adaptive (slice bounds from the launches' feedback)
  float adapt_gain;   // decode_bounds_kernel: fraction of the way to the measured shares a step moves
  int untimed;  // host only: never stamp this launch with timing events
#ifdef S8KV_DECODE_TRACE
  unsigned long long* trace;  // [grid][kTraceWords] per-workgroup records, or null
#endif
};

__device__ __forceinline__ int row_len(const DecodeArgs& a, int b) {
  return max(0, min(a.context_lens[b], a.max_context_len));
}
__device__ __forceinline__ int padded32(int n) { return (n + 31) & ~31; }

// Length of row b's part of the token stream: its tokens padded to a multiple
// of 32, plus `ghost` tokens that stand for a segment's fixed costs (q set-up,
// merge) so that slices holding row starts get fewer real tokens.  Empty rows
// take no space.
__device__ __forceinline__ int stream_len(const DecodeArgs& a, int L) { return L > 0 ? padded32(L) + a.ghost : 0; }

// Slices of a head's token stream, one per workgroup j of the head.
// Workgroups fill the CUs' residency slots in index order (class
// c = j * classes / W is the slot), and waves of later-dispatched workgroups
// lose instruction issue to older ones on the same CU, so a slot-c slice is
// weighted by 1 + skew * (classes - 1 - 2c) / (classes - 1).  Slice lengths
// are multiples of 32; the last slice runs to the end of the stream.
__device__ __forceinline__ int slot_first(int c, int W, int classes) { return (c * W + classes - 1) / classes; }
__device__ __forceinline__ float slot_weight(int c, int classes, int skew_permille) {
  return classes > 1 ? 1.0f + 0.001f * (float)(skew_permille * (classes - 1 - 2 * c) / (classes - 1)) : 1.0f;
}
// The slice layout is computed across lanes, lane c describing class c (at
// most 8 classes): every wave of every workgroup computes it, and scalar code
// doing the same would queue on the CU's one scalar unit.  Its cross-lane
// steps are swizzles and DPP row shifts, which need no lane-address
// registers, so the copy recomputed for a merge shares nothing with the
// prologue's.
template <int M>
__device__ __forceinline__ float swz_xor_f(float v) {  // lane ^ M, M < 32 (ds_swizzle bit mode)
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (M << 10)));
}
struct SliceLayout {
  int f0, f1;   // lane c: workgroups [f0, f1) are in class c (f0 = f1 = W past the last class)
  int sz;       // lane c: slice length of class c
  int start;    // lane c: stream position of class c's first slice
};
__device__ __forceinline__ SliceLayout slice_layout(int total, int W, int ncls, int skew_permille, int lane) {
  const int classes = max(1, min(ncls, min(W, kMaxResidentPerCU)));
  const bool act = lane < classes;
  SliceLayout s;
  s.f0 = act ? slot_first(lane, W, classes) : W;
  s.f1 = act ? slot_first(lane + 1, W, classes) : W;
  const float wt = act ? slot_weight(lane, classes, skew_permille) : 0.0f;
  float ws = (float)(s.f1 - s.f0) * wt;  // lanes 0..7 sum in a fixed tree order
  ws += swz_xor_f<1>(ws);
  ws += swz_xor_f<2>(ws);
  ws += swz_xor_f<4>(ws);
  const float wsum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ws), 0));
  const float unit = (float)total / wsum;
  s.sz = act ? max(kTile, padded32((int)ceilf(unit * wt))) : 0;
  const int span = (s.f1 - s.f0) * s.sz;
  int incl = span;  // inclusive scan over lanes 0..7 (DPP row_shr: lanes below `off` read 0)
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xF, 0xF, false);
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, false);
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, false);
  s.start = incl - span;
  return s;
}
// Stream position where workgroup j's slice starts (0 <= j < W).
__device__ __forceinline__ int slice_start(const SliceLayout& s, int j) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(s.f0 <= j && j < s.f1);
  const int cl = m ? (int)__builtin_ctzll(m) : 0;
  return __builtin_amdgcn_readlane(s.start + (j - s.f0) * s.sz, cl);
}
// The workgroup whose slice holds stream position p (0 <= p < stream total):
// the largest j with slice_start(j) <= p.  Class starts increase with the
// class and the class spans cover the stream, so the last class starting at
// or before p holds it.
__device__ __forceinline__ int slice_of(const SliceLayout& s, int p) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(s.f0 < s.f1 && s.start <= p);
  const int cl = m ? 63 - (int)__builtin_clzll(m) : 0;
  const int k = min((p - s.start) / max(s.sz, 1), s.f1 - s.f0 - 1);
  return __builtin_amdgcn_readlane(s.f0 + k, cl);
}


// Inclusive prefix sum over the 64 lanes of a wave in DPP steps (VALU, no
// LDS round trips): shifts by 1, 2, 4, 8 within each 16-lane row (lanes
// shifted in from outside the row read 0), then lane 15 of rows 0 and 2 is
// added to rows 1 and 3, and lane 31 to rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return v;
}

// Context length of row b (clamped to [0, max_context_len]) from the LDS copy
// of the first kLensLds rows' context_lens entries.
__device__ __forceinline__ int lens_at(const DecodeArgs& a, const int* lens_lds, int b) {
  return b < kLensLds ? max(0, min(lens_lds[b], a.max_context_len)) : row_len(a, b);
}
// The unclamped context_lens entry of row b.
__device__ __forceinline__ int raw_len_at(const DecodeArgs& a, const int* lens_lds, int b) {
  return b < kLensLds ? lens_lds[b] : a.context_lens[b];
}

// Checksum of the raw context lengths (a plan records the one of the lengths
// it was made from; a planned launch recomputes it and ignores a plan whose
// lengths were changed in place since).  Every lane returns the same value.
__device__ __forceinline__ uint32_t lens_checksum(const DecodeArgs& a, const int* lens_lds, int lane) {
  uint32_t s = 0;
  for (int c0 = 0; c0 < a.batch; c0 += 64) {
    const int b = c0 + lane;
    const uint32_t v =
        b < a.batch ? ((uint32_t)raw_len_at(a, lens_lds, b) + 1u) * (2u * (uint32_t)b + 1u) * 0x9E3779B1u : 0u;
    s += (uint32_t)__builtin_amdgcn_readlane(wave_incl_scan((int)v), 63);
  }
  return s;
}
constexpr int kPlanLensWord = 15;  // header word holding lens_checksum

// Sliding window: a row of L tokens attends positions [L - window, L); the
// kernel views it from win_base, that start rounded down to a multiple of 32
// (so its tiles stay 32-aligned in the block table), and masks the tokens of
// the first tile below the start.
__device__ __forceinline__ int win_base(const DecodeArgs& a, int L) { return max(0, L - a.window) & ~31; }
// Tokens of row b the kernel streams: all of them, or those from win_base on.
template <bool WIN>
__device__ __forceinline__ int view_len(const DecodeArgs& a, const int* lens_lds, int b) {
  const int L = lens_at(a, lens_lds, b);
  if constexpr (WIN) return L - win_base(a, L);
  return L;
}

// Stream length of rows c0 + lane (0 past the batch).
template <bool WIN>
__device__ __forceinline__ int row_stream_len(const DecodeArgs& a, const int* lens_lds, int c0, int lane) {
  const int r = c0 + lane;
  return r < a.batch ? stream_len(a, view_len<WIN>(a, lens_lds, r)) : 0;
}

// ---- where a workgroup's work lies ----
// The slice of workgroup column j in its head's token stream and the segment
// it processes first.  Every decode launch can compute it from the context
// lengths in its prologue; the launches of one step (one per layer, the same
// lengths and block table) can instead share one plan computed once by
// decode_plan_kernel (s8kv_decode_plan), whose entry for column j also holds
// the storage row (KV head 0) of each wave's first tile, so that a planned
// launch issues its first K/V loads before anything else.
struct SliceLoc {
  int total;                       // the head's stream length
  int lo, hi;                      // the slice [lo, hi)
  int b, pb, L;                    // the segment processed first: row, its stream start, its length (0: none)
  int b_first, pb_first, L_first;  // the slice's first segment
  int b_stop;                      // rows from here on are left to the reordered segment
  int reordered;                   // the slice's last segment runs first
};
// Plan layout (int32 words): a header naming the launch geometry the plan was
// made for, then one entry per workgroup column j.
constexpr int kPlanHeader = 32;       // words before the entries (entries stay 64-byte aligned)
constexpr int kPlanHeaderWords = 17;  // header words in use
constexpr int kPlanEntry = 16;
constexpr int kPlanMagic = 0x50384B53;
constexpr int kPlanAdaptWord = 16;  // header word: 1 when the slice bounds come from the adaptive area
// Adaptive plans (s8kv_decode_plan_adaptive) keep, after the entries, the
// slice bounds they were made with and the launches' feedback: every
// workgroup (column j, KV head h) of a launch reading the plan records its
// run time and slice length there, tagged with the plan's epoch, and the
// next step's plan moves the bounds towards equal run times.
constexpr int kAdaptMagic = 0x41445053;
enum AdaptWord { kAdMagic = 0, kAdWg, kAdHkv, kAdBatch, kAdEpoch, kAdTotal, kAdBounds = 8 };
constexpr int kFbWords = 3;  // feedback entry (KV head h, column j): epoch, start and end (s_memrealtime, low words)
__host__ __device__ inline int64_t plan_adapt_off(int wmax) { return kPlanHeader + (int64_t)kPlanEntry * wmax; }
__host__ __device__ inline int64_t plan_fb_off(int wmax) { return plan_adapt_off(wmax) + kAdBounds + wmax + 1; }
constexpr uint32_t kNoTile = 0xFFFFFFFFu;
// Word i of a plan, read through the constant address space so that a
// wave-uniform index becomes a scalar load: the decode prologue's header,
// entry and epoch reads are then issued together instead of as a chain of
// vector loads each waited on before the next (the decode launch writes only
// the plan's feedback words, which it never reads).
using plan_word_t = const __attribute__((address_space(4))) int32_t;
__device__ __forceinline__ int32_t plan_word(const int32_t* plan, int64_t i) {
  return ((plan_word_t*)plan)[i];  // (an address-space cast: C-style)
}
enum PlanWord {  // entry words
  kPwTotal = 0, kPwLo, kPwHi, kPwB, kPwPb, kPwL, kPwBFirst, kPwPbFirst, kPwLFirst, kPwBStop, kPwReordered,
  kPwTile0 = 12,  // kPwTile0 + w: wave w's first tile row at KV head 0, or kNoTile
};
// Header word i of the plan a launch with arguments `a` needs.
__host__ __device__ inline int32_t plan_header_word(const DecodeArgs& a, int i) {
  switch (i) {
    case 0: return kPlanMagic;
    case 1: return a.batch;
    case 2: return a.max_context_len;
    case 3: return a.wg_per_head;
    case 4: return a.slot_classes;
    case 5: return a.slot_skew;
    case 6: return a.ghost;
    case 7: return a.bs_log2;
    case 8: return a.num_kv_heads;
    case 9: return a.window;
    case 10: return (int32_t)(uint32_t)(uintptr_t)a.block_table;
    case 11: return (int32_t)(uint32_t)((uint64_t)(uintptr_t)a.block_table >> 32);
    case 12: return (int32_t)(uint32_t)(uintptr_t)a.context_lens;
    case 13: return (int32_t)(uint32_t)((uint64_t)(uintptr_t)a.context_lens >> 32);
    case 14: return (int32_t)a.bt_stride;
    default: return 0;
  }
}

// Advance (rb, rpb) to the first row from rb on whose real tokens
// [rpb + ghost, rpb + ghost + padded32(L)) overlap [lo, hi); returns its
// length, or 0 when the slice holds no further segment.
template <bool WIN>
__device__ __forceinline__ int find_segment(const DecodeArgs& a, const int* lens_lds, int lo, int hi, int& rb,
                                            int& rpb) {
  for (; rb < a.batch && rpb + a.ghost < hi; ++rb) {
    const int L = __builtin_amdgcn_readfirstlane(view_len<WIN>(a, lens_lds, rb));
    if (L == 0) continue;
    if (rpb + a.ghost + padded32(L) > lo) return L;
    rpb += stream_len(a, L);
  }
  return 0;
}

// The head's stream length (every lane).
template <bool WIN>
__device__ __forceinline__ int stream_total(const DecodeArgs& a, const int* lens_lds, int lane) {
  int total = 0;
  for (int c0 = 0; c0 < a.batch; c0 += 64)
    total += __builtin_amdgcn_readlane(wave_incl_scan(row_stream_len<WIN>(a, lens_lds, c0, lane)), 63);
  return __builtin_amdgcn_readfirstlane(total);
}
template <bool WIN>
__device__ __forceinline__ bool slice_segments(const DecodeArgs& a, const int* lens_lds, int lane, SliceLoc& s);
// Column j's slice and the segment it processes first, from the context
// lengths in LDS (all lanes of a wave; the results are wave-uniform).
// Returns false when the slice holds no segment.
template <bool WIN>
__device__ __forceinline__ bool locate_slice(const DecodeArgs& a, const int* lens_lds, int j, int lane, SliceLoc& s) {
  s.total = stream_total<WIN>(a, lens_lds, lane);
  s.L = 0;
  const SliceLayout sl = slice_layout(s.total, a.wg_per_head, a.slot_classes, a.slot_skew, lane);
  s.lo = slice_start(sl, j);
  if (s.lo >= s.total) return false;
  s.hi = j + 1 >= a.wg_per_head ? s.total : min(s.total, slice_start(sl, j + 1));
  return slice_segments<WIN>(a, lens_lds, lane, s);
}
// The first segment (and the segment order) of the slice [s.lo, s.hi) of a
// stream of s.total tokens; false when the slice holds no segment.
template <bool WIN>
__device__ __forceinline__ bool slice_segments(const DecodeArgs& a, const int* lens_lds, int lane, SliceLoc& s) {
  s.L = 0;
  if (s.lo >= s.hi) return false;
  const int v0 = row_stream_len<WIN>(a, lens_lds, 0, lane);
  const int incl0 = wave_incl_scan(v0);  // rows 0..63

  // the row whose stream range holds position pos (< total), and the start of that range
  auto find_row = [&](int pos, int& rb, int& rpb) {
    rb = 0;
    rpb = 0;
    int carry = 0;
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
      const int v = c0 == 0 ? v0 : row_stream_len<WIN>(a, lens_lds, c0, lane);
      const int incl = (c0 == 0 ? incl0 : wave_incl_scan(v)) + carry;
      const uint64_t m = __builtin_amdgcn_ballot_w64(incl > pos);
      if (m != 0) {
        const int f = (int)__builtin_ctzll(m);
        rb = c0 + f;
        rpb = __builtin_amdgcn_readlane(incl - v, f);
        break;
      }
      carry = __builtin_amdgcn_readlane(incl, 63);
    }
    rb = __builtin_amdgcn_readfirstlane(rb);
    rpb = __builtin_amdgcn_readfirstlane(rpb);
  };
  int b, pb;
  find_row(s.lo, b, pb);
  int L = find_segment<WIN>(a, lens_lds, s.lo, s.hi, b, pb);
  if (L == 0) return false;
  // Segment order: when the slice's last segment is split by the slice end
  // (its row continues in the next slice) and is not its first segment, it
  // is processed first, then the segments from the first one on, stopping
  // before its row.  Both parts of a row shared by two slices are then
  // processed early in their slices, so the row's combine happens while
  // other workgroups stream, not in the kernel's tail.
  s.b_first = b;
  s.pb_first = pb;
  s.L_first = L;
  s.b_stop = a.batch;
  s.reordered = 0;
  {
    int bl, pbl;
    find_row(s.hi - 1, bl, pbl);
    const int Ll = bl > b ? __builtin_amdgcn_readfirstlane(view_len<WIN>(a, lens_lds, bl)) : 0;
    if (Ll > 0 && pbl + a.ghost < s.hi && pbl + a.ghost + padded32(Ll) > s.hi) {
      b = bl;
      pb = pbl;
      L = Ll;
      s.b_stop = bl;
      s.reordered = 1;
    }
  }
  s.b = b;
  s.pb = pb;
  s.L = L;
  return true;
}

// Position of tile token tt (0..31) in the LDS-staged V tile: lane group g's
// eight transpose-read rows (tokens 4g..4g+3 and 16+4g..16+4g+3) are
// consecutive rows 8g..8g+7.
__device__ __forceinline__ int lds_row_of(int tt) { return 8 * ((tt & 15) >> 2) + 4 * (tt >> 4) + (tt & 3); }

template <int KCH, int AUX>
__device__ __forceinline__ void load_kchunk(rsrc_t r, uint32_t off, uint32_t (&dst)[KCH / 4], uint32_t soff = 0) {
  if constexpr (KCH == 8) {
    u32x2_t v = bload64<AUX>(r, off, soff);
    dst[0] = v.x; dst[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < KCH / 16; ++i) {
      u32x4_t v = bload128<AUX>(r, off + 16 * i, soff);
      dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
    }
  }
}

template <int D, bool K8V3>
struct TileIO {
  using C = DecCfg<D, K8V3>;
  uint32_t k[2][C::KCH / 4];        // K rows, MFMA A layout
  u32x4_t v[C::VLOADS];             // int8: 16-byte V chunks; K8V3: packed words (x,y,z used)
  float4_t ks[2];
  float4_t vs[2][C::NB];
};

template <int D, bool K8V3, bool FUSE, bool WIN = false, bool BIG = false>
__global__ __launch_bounds__(64 * kDecWaves, D >= 256 ? 2 : 3) void decode_kernel(DecodeArgs a) {
  static_assert(!(FUSE && WIN), "the sliding-window form has no fused append");
  using C = DecCfg<D, K8V3>;
  constexpr int E = RowLayout<D>::E;
  // LDS: [V staging of the 4 waves | rotated q; the cross-wave merge reuses both][block ids]
  //      [context lengths][fused append: the new token's rows]
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int* bt_lds = reinterpret_cast<int*>(smem + a.smem_main);
  int* lens_lds = bt_lds + kMaxSubBlocks;

  const uint32_t t_start = (uint32_t)__builtin_amdgcn_s_memrealtime();  // adaptive plans: this workgroup's start
  const int Hkv = a.num_kv_heads;
  const int h = blockIdx.x % Hkv;
  const int j = blockIdx.x / Hkv;
  const int G = a.group;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
#ifdef S8KV_DECODE_TRACE
  __shared__ unsigned long long trace_lds[kTraceWords];
  if (tid < kTraceWords) trace_lds[tid] = 0;
  __syncthreads();
  S8KV_TRACE_STAMP(kTrEntry);
  unsigned long long tr_tok = 0, tr_seg = 0;
#endif

  const rsrc_t kc = make_rsrc(a.k_cache, a.kc_bytes);
  const rsrc_t ks = make_rsrc(a.k_scale, a.ks_bytes);
  const rsrc_t vc = make_rsrc(a.v_cache, a.vc_bytes);
  const rsrc_t vs = make_rsrc(a.v_scale, a.vs_bytes);
  char* vstage = smem + wave * C::VSTAGE;
  const uint32_t hkv = (uint32_t)Hkv;
  const int bs_log2 = a.bs_log2;
  const uint32_t bsm = (1u << bs_log2) - 1u;
  // A 32-token tile never crosses a block when block_size >= 32: the tile's
  // first storage row is then wave-uniform and rides in the buffer loads'
  // scalar offset, while each lane's vector offset is a loop constant.
  const bool tile_in_block = bs_log2 >= 5;
  constexpr int LPR = D / 16;    // int8 V: lanes per 16-byte-chunked row
  constexpr int RPI = 64 / LPR;  // int8 V: rows per load instruction
  // block ids staged per segment start: the first sub-split's (at most kSubTokens tokens)
  const int bt_width = (a.max_context_len + (1 << bs_log2) - 1) >> bs_log2;  // readable entries per row
  const int bt_first = (kSubTokens >> bs_log2) + 1;
  constexpr int kBtRegs = (kMaxSubBlocks + 64 * kDecWaves - 1) / (64 * kDecWaves);
  constexpr int kPol = kTilePolicy<K8V3>;

  // The tile's loads in flight (a planned launch issues its first tile in the
  // prologue), and the loads of a tile inside one block (block_size >= 32)
  // from its first storage row r0: K and V, then the scales.
  TileIO<D, K8V3> io;
  auto tile_kv_at = [&](uint32_t r0, int ln) {
    const int cc = ln & 15, gg = ln >> 4;
    if constexpr (BIG) {  // descriptors rebased to the tile's first row
      const rsrc_t kt = window_rsrc(a.k_cache, a.kc_total, (uint64_t)r0 * D);
#pragma unroll
      for (int s = 0; s < 2; ++s) load_kchunk<C::KCH, kPol>(kt, (uint32_t)((16 * s + cc) * D + gg * C::KCH), io.k[s]);
      if constexpr (!K8V3) {
        const rsrc_t vt = window_rsrc(a.v_cache, a.vc_total, (uint64_t)r0 * D);
#pragma unroll
        for (int jj = 0; jj < C::VLOADS; ++jj)
          io.v[jj] = bload128<kPol>(vt, (uint32_t)((jj * RPI + ln / LPR) * D + (ln % LPR) * 16));
      } else {
        const rsrc_t vt = window_rsrc(a.v_cache, a.vc_total, (uint64_t)r0 * (C::WORDS * 4));
#pragma unroll
        for (int jj = 0; jj < C::VLOADS; ++jj) {
          const int job = jj * 64 + ln;
          const uint32_t off = (uint32_t)(((job / C::NG) * C::WORDS + (job % C::NG) * 3) * 4);
          const u32x3_t w = bload96<kPol>(vt, off);
          io.v[jj].x = w.x;
          io.v[jj].y = w.y;
          io.v[jj].z = w.z;
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s)
        load_kchunk<C::KCH, kPol>(kc, (uint32_t)((16 * s + cc) * D + gg * C::KCH), io.k[s], r0 * (uint32_t)D);
      if constexpr (!K8V3) {
#pragma unroll
        for (int jj = 0; jj < C::VLOADS; ++jj)
          io.v[jj] = bload128<kPol>(vc, (uint32_t)((jj * RPI + ln / LPR) * D + (ln % LPR) * 16), r0 * (uint32_t)D);
      } else {
#pragma unroll
        for (int jj = 0; jj < C::VLOADS; ++jj) {
          const int job = jj * 64 + ln;
          const uint32_t off = (uint32_t)(((job / C::NG) * C::WORDS + (job % C::NG) * 3) * 4);
          const uint32_t so = r0 * (uint32_t)(C::WORDS * 4);
          const u32x3_t w = bload96<kPol>(vc, off, so);
          io.v[jj].x = w.x;
          io.v[jj].y = w.y;
          io.v[jj].z = w.z;
        }
      }
    }
  };
  auto tile_scales_at = [&](uint32_t r0, int ln) {
    const int gg = ln >> 4;
    rsrc_t kst = ks, vst = vs;
    uint32_t so = r0;
    if constexpr (BIG) {
      kst = window_rsrc(a.k_scale, a.ks_total, (uint64_t)r0 * 4u);
      vst = window_rsrc(a.v_scale, a.vs_total, (uint64_t)r0 * (C::NB * 4u));
      so = 0;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t row = (uint32_t)(16 * s + 4 * gg);
      io.ks[s] = bloadf4<kPol>(kst, row * 4u, so * 4u);
      if constexpr (C::NB == 1) {
        io.vs[s][0] = bloadf4<kPol>(vst, row * 4u, so * 4u);
      } else {
        const float4_t n0 = bloadf4<kPol>(vst, row * 8u, so * 8u), n1 = bloadf4<kPol>(vst, row * 8u + 16u, so * 8u);
        io.vs[s][0] = float4_t{n0.x, n0.z, n1.x, n1.z};  // [token][block] -> per block
        io.vs[s][1] = float4_t{n0.y, n0.w, n1.y, n1.w};
      }
    }
  };

  // Set-up loads of a segment that starts at token 0 of row rb (or at s0 for
  // the slice's first row): the lane's raw q fragment and the first
  // sub-split's block ids, issued early so their latency overlaps other work.
  _Float16 qraw[kQHeadsPerWave][E];
  int btv[kBtRegs];
  _Float16 knr[E], vnr[E];  // fused append: row rb's new K and V (RowLayout lanes)
  auto prefetch_segment = [&](int rb, int s0) {
    if constexpr (FUSE) {
      const int lane_o = opaque_int(threadIdx.x) & 63;
      const _Float16* kp = a.k_new + (int64_t)rb * a.kn_stride_b + (int64_t)h * a.kn_stride_h;
      const _Float16* vp = a.v_new + (int64_t)rb * a.vn_stride_b + (int64_t)h * a.vn_stride_h;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const bool on = lane_o < RowLayout<D>::ACTIVE;
        knr[e] = on ? kp[lane_o + 64 * e] : (_Float16)0.0f;
        vnr[e] = on ? vp[lane_o + 64 * e] : (_Float16)0.0f;
      }
    }
    // q of this wave's heads c = wave + 4k (lane l: dims l + 64e), the heads
    // the wave rotates for the whole workgroup
    const int tid_o = opaque_int(threadIdx.x);
    const int lane_q = tid_o & 63;
#pragma unroll
    for (int k = 0; k < kQHeadsPerWave; ++k) {
      const int cq = wave + kDecWaves * k;
      const _Float16* qp = a.q + (int64_t)rb * a.q_stride_b + (int64_t)(h * G + (cq < G ? cq : 0)) * a.q_stride_h;
#pragma unroll
      for (int e = 0; e < E; ++e)
        qraw[k][e] = (cq < G && lane_q < RowLayout<D>::ACTIVE) ? qp[lane_q + 64 * e] : (_Float16)0.0f;
    }
    const int al = WIN ? win_base(a, __builtin_amdgcn_readfirstlane(lens_at(a, lens_lds, rb))) : 0;
    const int fb = (s0 + al) >> bs_log2;
    const int32_t* bt_row = a.block_table + (int64_t)rb * a.bt_stride + fb;
#pragma unroll
    for (int k = 0; k < kBtRegs; ++k) {
      const int i = tid_o + k * 64 * kDecWaves;
      btv[k] = (i < bt_first && fb + i < bt_width) ? bt_row[i] : 0;
    }
  };
  auto store_prefetched_bt = [&]() {
    const int tid_o = opaque_int(threadIdx.x);
#pragma unroll
    for (int k = 0; k < kBtRegs; ++k) {
      const int i = tid_o + k * 64 * kDecWaves;
      if (i < bt_first) bt_lds[i] = btv[k];
    }
  };
  // q: each wave rotates the heads c = wave + 4k of the group (lane l holds
  // dims l + 64e: the append's fp32 FWHT, stages h = 1 .. D/2 in order),
  // splits the scaled values into fp16 hi + lo and publishes them in LDS
  // ([hi, lo][G][D]; a barrier later, every wave takes its MFMA B fragments)
  auto publish_q = [&]() {
    const int lane_q = opaque_int(threadIdx.x) & 63;
    _Float16* qs = reinterpret_cast<_Float16*>(smem + C::SMEM_Q);
#pragma unroll
    for (int k = 0; k < kQHeadsPerWave; ++k) {
      const int cq = wave + kDecWaves * k;
      if (cq < G) {
        float x[E];
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = (float)qraw[k][e];
        fwht_row<D>(x, lane_q);
        if (lane_q < RowLayout<D>::ACTIVE) {
#pragma unroll
          for (int e = 0; e < E; ++e) {
            // (materialized: hi and lo must both come from this one fp32 value;
            // a fused fp16(x*s) for the lo term can differ from fp16(val) by one
            // ulp, which would leave hi + lo off by 2^-11)
            const float val = materialize(x[e] * a.qscale);
            const _Float16 qh = (_Float16)val;
            qs[cq * D + lane_q + 64 * e] = qh;
            qs[(G + cq) * D + lane_q + 64 * e] = (_Float16)(val - (float)qh);
          }
        }
      }
    }
  };

  // context lengths, loaded first so that they return ahead of the set-up and
  // tile loads issued below (one global round trip for the whole prologue)
  constexpr int kLensRegs = kLensLds / (64 * kDecWaves);
  const int n_lens = min(a.batch, kLensLds);
  int lens_r[kLensRegs];
#pragma unroll
  for (int k = 0; k < kLensRegs; ++k) {
    const int i = tid + k * 64 * kDecWaves;
    lens_r[k] = i < n_lens ? a.context_lens[i] : 0;
  }

  // ---- the slice and its first segment: from the step's plan, or located here ----
  SliceLoc sl;
  bool q_ready = false;  // the first segment's rotated q is published (planned prologue)
  bool pre_issued = false;  // this wave's first tile of the first segment is in flight
  uint32_t pre_r0 = kNoTile;  // ... from this storage row
  bool planned = false;
  bool adapt = false;  // the plan's slices come from its adaptive bounds: record this workgroup's times
  int epoch = 0;
  int32_t ew[kPlanEntry];  // this column's plan entry
  int32_t plan_lens_cs = 0;  // the plan's lens_checksum
  if (a.plan != nullptr) {
    // every plan word the prologue reads, loaded together (the host checked
    // that the buffer holds the whole layout): no chain of dependent loads
    planned = true;
#pragma unroll
    for (int i = 0; i < kPlanHeaderWords; ++i)
      planned &= i == kPlanLensWord || i == kPlanAdaptWord || plan_word(a.plan, i) == plan_header_word(a, i);
    const int32_t aw = plan_word(a.plan, kPlanAdaptWord);
    plan_lens_cs = plan_word(a.plan, kPlanLensWord);
    const int32_t ep = plan_word(a.plan, plan_adapt_off(a.plan_wmax) + kAdEpoch);
#pragma unroll
    for (int i = 0; i < kPlanEntry; ++i) ew[i] = plan_word(a.plan, kPlanHeader + (int64_t)j * kPlanEntry + i);
    adapt = planned && aw == 1;
    epoch = ep;
  }
  // the workgroup's times, tagged with the plan's epoch (thread 0, at the workgroup's end)
  auto record_times = [&]() {
    if (adapt && tid == 0) {
      int32_t* f = const_cast<int32_t*>(a.plan) + plan_fb_off(a.plan_wmax) + ((int64_t)h * a.plan_wmax + j) * kFbWords;
      f[0] = epoch;
      f[1] = (int32_t)t_start;
      f[2] = (int32_t)(uint32_t)__builtin_amdgcn_s_memrealtime();
    }
  };
  uint32_t r0 = kNoTile;  // this wave's first tile row at KV head 0, from the plan
  if (planned) {
    sl.total = ew[kPwTotal];
    sl.lo = ew[kPwLo];
    sl.hi = ew[kPwHi];
    sl.b = ew[kPwB];
    sl.pb = ew[kPwPb];
    sl.L = ew[kPwL];
    sl.b_first = ew[kPwBFirst];
    sl.pb_first = ew[kPwPbFirst];
    sl.L_first = ew[kPwLFirst];
    sl.b_stop = ew[kPwBStop];
    sl.reordered = ew[kPwReordered];
    r0 = (uint32_t)(wave == 0 ? ew[kPwTile0] : wave == 1 ? ew[kPwTile0 + 1]
                    : wave == 2 ? ew[kPwTile0 + 2] : ew[kPwTile0 + 3]);
    // (rows outside the batch would index outputs and partials out of range)
    if (sl.L > 0 && !(sl.b >= 0 && sl.b < a.batch && sl.b_first >= 0 && sl.b_first < a.batch && sl.b_stop >= 0 &&
                      sl.b_stop <= a.batch))
      planned = false;
  }
  auto stage_lens = [&]() {
#pragma unroll
    for (int k = 0; k < kLensRegs; ++k) {
      const int i = tid + k * 64 * kDecWaves;
      if (i < n_lens) lens_lds[i] = lens_r[k];
    }
    __syncthreads();
    S8KV_TRACE_STAMP(kTrLens);
  };
  // a plan made from other lengths (the buffer rewritten in place since) is
  // ignored; a first tile issued from it is issued again below when its row differs
  if (!WIN && planned && sl.L > 0 && tile_in_block) {
    // planned prologue, straight-line so that each wait covers only what it
    // needs: the first segment's set-up loads (q, block ids, the new token's
    // rows), then this wave's first tile (storage row 0 as a stand-in when the
    // wave has none, so that every wave has the same loads in flight), then
    // the lengths (loaded first) -> LDS, the plan's checksum, the block ids
    // -> LDS and q rotated and published while the tile is in flight
    prefetch_segment(sl.b, max(sl.lo, sl.pb + a.ghost) - (sl.pb + a.ghost));
    const uint32_t rr = r0 != kNoTile ? r0 + ((uint32_t)h << bs_log2) : 0u;
    tile_kv_at(rr, lane);
    tile_scales_at(rr, lane);
    pre_issued = r0 != kNoTile;
    pre_r0 = rr;
    stage_lens();
    if ((int32_t)lens_checksum(a, lens_lds, lane) == plan_lens_cs) {
      store_prefetched_bt();
      publish_q();
      q_ready = true;
    } else {
      planned = false;
    }
  } else {
    stage_lens();
    if (planned && (int32_t)lens_checksum(a, lens_lds, lane) != plan_lens_cs) planned = false;
  }
  adapt = adapt && planned;
  bool has_seg = planned ? sl.L > 0 : locate_slice<WIN>(a, lens_lds, j, lane, sl);
  if (j == 0) {  // empty rows attend nothing: their output is defined as zeros
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
      uint64_t m = __builtin_amdgcn_ballot_w64(c0 + lane < a.batch && lens_at(a, lens_lds, c0 + lane) == 0);
      while (m != 0) {
        const int b = c0 + (int)__builtin_ctzll(m);
        m &= m - 1;
        for (int i = tid; i < G * D; i += 64 * kDecWaves)
          a.out[((int64_t)b * a.num_q_heads + h * G) * D + i] = (_Float16)0.0f;
      }
    }
  }
  if (!has_seg) {
    record_times();
    return;
  }
  const int total = sl.total, lo = sl.lo, hi = sl.hi;

  // K8V3 codebook byte tables (fp16 of the fp32 codebook).
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

  int b = sl.b, pb = sl.pb, L = sl.L;
  const int b_first = sl.b_first, pb_first = sl.pb_first, L_first = sl.L_first;
  const int b_stop = sl.b_stop;  // rows from here on are left to the reordered segment
  bool reordered = sl.reordered != 0;
  S8KV_TRACE_STAMP(kTrFound);
  if (!q_ready) {
    prefetch_segment(b, max(lo, pb + a.ghost) - (pb + a.ghost));
    store_prefetched_bt();
  }
  S8KV_TRACE_STAMP(kTrStaged);

  // ---- segments: rows overlapping [lo, hi) ----
  for (;;) {
    __syncthreads();  // staged block ids visible; the previous merge is done with LDS
    // per-lane values of this segment's q set-up and merge, from an opaque
    // copy of the thread id (see the tile loop below)
    const int tid = opaque_int(threadIdx.x);
    const int lane = tid & 63;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int padL = padded32(L);
    const int rs = pb + a.ghost;              // stream position of the row's token 0
    const int s0 = max(lo, rs) - rs;          // segment [s0, s1) in row coordinates
    const int s1 = min(hi, rs + padL) - rs;   // multiples of 32; s0 < L
    const bool whole_row = (s0 == 0) && (s1 == padL);
    const int last = L - 1;
    const int32_t* bt_row = a.block_table + (int64_t)b * a.bt_stride;
    // sliding window: row coordinates start at absolute position al; tokens
    // below lo_tok (in the row's first tile) are outside the window
    int al = 0, lo_tok = 0;
    if constexpr (WIN) {
      const int Lf = __builtin_amdgcn_readfirstlane(lens_at(a, lens_lds, b));
      al = win_base(a, Lf);
      lo_tok = max(0, Lf - a.window) - al;
    }

    // q rotated and published (the planned prologue did the first segment's),
    // then every wave takes its MFMA B fragments (lane (c, g): dims
    // g*KCH + 8m .. +8 of head c)
    if (!q_ready) publish_q();
    q_ready = false;
    const _Float16* qs = reinterpret_cast<const _Float16*>(smem + C::SMEM_Q);  // [hi, lo][G][D]
    __syncthreads();  // every head of q published
    S8KV_TRACE_STAMP_ONCE(kTrQ);
    half8_t qhi[C::NQK], qlo[C::NQK];
#pragma unroll
    for (int m = 0; m < C::NQK; ++m) {
      qhi[m] = c < G ? *reinterpret_cast<const half8_t*>(qs + c * D + g * C::KCH + 8 * m) : half8_t{};
      qlo[m] = c < G ? *reinterpret_cast<const half8_t*>(qs + (G + c) * D + g * C::KCH + 8 * m) : half8_t{};
    }

    // fused append: the wave that will process the row's last tile keeps the
    // new token's fp16 rows in LDS until that tile (its registers are needed
    // by the tile loop)
    const int raw_len = raw_len_at(a, lens_lds, b);
    const bool app_seg = FUSE && raw_len >= 1 && raw_len <= a.max_context_len && s1 == padL;
    if constexpr (FUSE) {
      const int u_last = s0 + ((s1 - 1 - s0) / kSubTokens) * kSubTokens;
      if (app_seg && wave == ((padL - kTile - u_last) / kTile) % kDecWaves) {
        _Float16* nf = reinterpret_cast<_Float16*>(smem + a.smem_new + C::NEW_F16K);
        if (lane < RowLayout<D>::ACTIVE) {
#pragma unroll
          for (int e = 0; e < E; ++e) {
            nf[lane + 64 * e] = knr[e];
            nf[D + lane + 64 * e] = vnr[e];  // NEW_F16V = 2D bytes on
          }
        }
      }
    }

    float m_ref = kNegInf;  // running max - esh (WeightShift)
    float l_run = 0.0f;
    WeightShift ws(kMaxSlack);
    float4_t acc[C::NPV];
#pragma unroll
    for (int n = 0; n < C::NPV; ++n) acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};

    // ---- sub-splits of <= kSubTokens tokens; the first one's block ids are staged ----
    for (int u0 = s0; u0 < s1; u0 += kSubTokens) {
      const int u1 = min(s1, u0 + kSubTokens);
      const int t1 = min(u1, L);               // valid tokens end
      const int fb = (u0 + al) >> bs_log2;     // block-table index of the sub-split's first block
      // Lane-derived addresses of the tile loop are recomputed per sub-split:
      // the opaque copy of the thread id stops the compiler from hoisting them
      // out of the segment loop, where they would stay live across the q
      // set-up and the merge and cost a wave per SIMD of occupancy.
      const int lane = opaque_int(tid) & 63;  // shadows the segment's lane, c, g
      const int c = lane & 15;
      const int g = lane >> 4;
      if (u0 != s0) {  // later sub-splits of a long segment: stage their block ids now
        const int nblk = ((t1 - 1 + al) >> bs_log2) - fb + 1;
        __syncthreads();
        for (int i = tid; i < nblk; i += 64 * kDecWaves) bt_lds[i] = bt_row[fb + i];
        __syncthreads();
      }

      // storage row of token `tok` (already clamped to the row's last token)
      auto row_of = [&](int tok) -> uint32_t {
        if constexpr (WIN) tok += al;
        const uint32_t blk = (uint32_t)bt_lds[(tok >> bs_log2) - fb];
        return ((blk * hkv + (uint32_t)h) << bs_log2) + ((uint32_t)tok & bsm);
      };
      auto tile_row0 = [&](int tb) -> uint32_t {
        if constexpr (WIN) tb += al;
        const uint32_t blk = (uint32_t)bt_lds[(tb >> bs_log2) - fb];
        return __builtin_amdgcn_readfirstlane(((blk * hkv + (uint32_t)h) << bs_log2) + ((uint32_t)tb & bsm));
      };

      auto issue_kv = [&](int tb, uint32_t r0) {
        if (BIG || tile_in_block) {  // (BIG needs block_size >= 32)
          tile_kv_at(r0, lane);
          return;
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const uint32_t row = row_of(min(tb + 16 * s + c, last));
          load_kchunk<C::KCH, kPol>(kc, row * (uint32_t)D + (uint32_t)(g * C::KCH), io.k[s]);
        }
        if constexpr (!K8V3) {
#pragma unroll
          for (int jj = 0; jj < C::VLOADS; ++jj) {
            const uint32_t row = row_of(min(tb + jj * RPI + lane / LPR, last));
            io.v[jj] = bload128<kPol>(vc, row * (uint32_t)D + (uint32_t)((lane % LPR) * 16));
          }
        } else {
#pragma unroll
          for (int jj = 0; jj < C::VLOADS; ++jj) {
            const int job = jj * 64 + lane;
            const uint32_t row = row_of(min(tb + job / C::NG, last));
            const uint32_t base = row * (uint32_t)(C::WORDS * 4) + (uint32_t)((job % C::NG) * 12);
            const u32x3_t w = bload96<kPol>(vc, base);
            io.v[jj].x = w.x;
            io.v[jj].y = w.y;
            io.v[jj].z = w.z;
          }
        }
      };
      auto issue_scales = [&](int tb, uint32_t r0) {
        if (BIG || tile_in_block) {
          tile_scales_at(r0, lane);
          return;
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const uint32_t row = row_of(min(tb + 16 * s + 4 * g, last & ~3));
          io.ks[s] = bloadf4<kPol>(ks, row * 4u);
          if constexpr (C::NB == 1) {
            io.vs[s][0] = bloadf4<kPol>(vs, row * 4u);
          } else {
            const float4_t n0 = bloadf4<kPol>(vs, row * 8u), n1 = bloadf4<kPol>(vs, row * 8u + 16u);
            io.vs[s][0] = float4_t{n0.x, n0.z, n1.x, n1.z};  // [token][block] -> per block
            io.vs[s][1] = float4_t{n0.y, n0.w, n1.y, n1.w};
          }
        }
      };

      // One 32-token tile: MASKED only for a wave's last tile of the sub-split
      // (may run past t1); PREFETCH issues the loads of the wave's next tile,
      // which then always exists.
      auto process = [&](int tb, auto masked_tag, auto prefetch_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        constexpr bool PREFETCH = decltype(prefetch_tag)::value;
        const int tn = tb + kTile * kDecWaves;
        uint32_t rn = 0;

        // 0. fused append: the row's last tile takes the new token's values
        // from the LDS rows the appending wave wrote (the loads may predate
        // the cache store)
        if constexpr (FUSE && MASKED) {
          if (app_seg && tb == padL - kTile) {
            const int r = last - tb;  // tile row of the new token
            const char* nn = smem + a.smem_new;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
              if (16 * s + c == r) {
#pragma unroll
                for (int w = 0; w < C::KCH / 4; ++w)
                  io.k[s][w] = *reinterpret_cast<const uint32_t*>(nn + C::NEW_I8K + g * C::KCH + 4 * w);
              }
            }
            if constexpr (!K8V3) {
#pragma unroll
              for (int jj = 0; jj < C::VLOADS; ++jj)
                if (jj * RPI + lane / LPR == r)
                  io.v[jj] = *reinterpret_cast<const u32x4_t*>(nn + C::NEW_V + (lane % LPR) * 16);
            } else {
              const uint32_t* nw = reinterpret_cast<const uint32_t*>(nn + C::NEW_V);
#pragma unroll
              for (int jj = 0; jj < C::VLOADS; ++jj) {
                const int job = jj * 64 + lane;
                if (job / C::NG == r) {
                  const int gi = job % C::NG;
                  io.v[jj].x = nw[3 * gi];
                  io.v[jj].y = nw[3 * gi + 1];
                  io.v[jj].z = nw[3 * gi + 2];
                }
              }
            }
            const float nks = *reinterpret_cast<const float*>(nn + C::NEW_KS);
            const float* nvs = reinterpret_cast<const float*>(nn + C::NEW_VS);
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                if (16 * s + 4 * g + i == r) {
                  io.ks[s][i] = nks;
#pragma unroll
                  for (int nb = 0; nb < C::NB; ++nb) io.vs[s][nb][i] = nvs[nb];
                }
              }
            }
          }
        }

        // 1. V tile -> LDS (int8 rows, or K8V3 codes expanded to fp16 rows)
        if constexpr (!K8V3) {
#pragma unroll
          for (int jj = 0; jj < C::VLOADS; ++jj) {
            const int tt = jj * RPI + lane / LPR;
            *reinterpret_cast<u32x4_t*>(vstage + lds_row_of(tt) * C::VROW + (lane % LPR) * 16) = io.v[jj];
          }
        } else {
#pragma unroll
          for (int jj = 0; jj < C::VLOADS; ++jj) {
            const int job = jj * 64 + lane;
            const int tt = job / C::NG, gi = job % C::NG;
            const uint32_t w0 = io.v[jj].x, w1 = io.v[jj].y, w2 = io.v[jj].z;
            char* dst = vstage + lds_row_of(tt) * C::VROW + gi * 64;
#pragma unroll
            for (int q4 = 0; q4 < 8; q4 += 2) {
              u32x4_t o;
              {
                const int i = 4 * q4;
                const uint32_t sel = spread4(w0 >> i) | (spread4(w1 >> i) << 1) | (spread4(w2 >> i) << 2);
                const u32x2_t r = codebook_lookup4(sel, tlo03, tlo47, thi03, thi47);
                o.x = r.x; o.y = r.y;
              }
              {
                const int i = 4 * q4 + 4;
                const uint32_t sel = spread4(w0 >> i) | (spread4(w1 >> i) << 1) | (spread4(w2 >> i) << 2);
                const u32x2_t r = codebook_lookup4(sel, tlo03, tlo47, thi03, thi47);
                o.z = r.x; o.w = r.y;
              }
              *reinterpret_cast<u32x4_t*>(dst + q4 * 8) = o;
            }
          }
        }

        // 2. QK
        float4_t sc[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          float4_t cacc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int m = 0; m < C::NQK; ++m) {
            const half8_t ka = i8x8_to_f16(u32x2_t{io.k[s][2 * m], io.k[s][2 * m + 1]});
            cacc = mfma16x16x32(ka, qhi[m], cacc);
            cacc = mfma16x16x32(ka, qlo[m], cacc);
          }
          sc[s] = cacc;
        }

        // 3. prefetch the next tile's K and V
        if constexpr (PREFETCH) {
          if (tile_in_block) rn = tile_row0(tn);
          issue_kv(tn, rn);
        }

        // 4. online softmax (log2 domain; q carries scale*log2e).  The running
        // max is raised lazily: only when some head's tile max exceeds it by
        // more than kMaxSlack, so p <= 2^(kMaxSlack + esh) and most tiles skip
        // the accumulator rescale.  First the weight shift: a V scale above
        // the bound lowers esh (WeightShift).
        {
          float vmx = 0.0f;
#pragma unroll
          for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int nb = 0; nb < C::NB; ++nb) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                float v = io.vs[s][nb][i];
                if constexpr (MASKED) {  // scales past the row end may be any value
                  const int tok = tb + 16 * s + 4 * g + i;
                  v = (tok < t1 && (!WIN || tok >= lo_tok)) ? v : 0.0f;
                }
                vmx = fmaxf(vmx, v);
              }
            }
          }
          if (__builtin_amdgcn_ballot_w64(vmx > ws.vbound()) != 0) {
            const int d = ws.raise(max_x32(max_x16(vmx)), kMaxSlack);
            const float f = __builtin_ldexpf(1.0f, d);
            l_run *= f;
#pragma unroll
            for (int n = 0; n < C::NPV; ++n) acc[n] *= f;
            m_ref -= (float)d;
          }
        }
        float p[2][4];
        float mt = kNegInf;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float x = sc[s][i] * io.ks[s][i];
            if constexpr (MASKED) {
              const int tok = tb + 16 * s + 4 * g + i;
              x = (tok < t1 && (!WIN || tok >= lo_tok)) ? x : kNegInf;
            }
            p[s][i] = x;
            mt = fmaxf(mt, x);
          }
        }
        mt = max_x16(mt);
        mt = max_x32(mt);
        if (__builtin_amdgcn_ballot_w64(mt > m_ref + ws.thr()) != 0) {
          const float m_new = fmaxf(m_ref, mt - (float)ws.esh);
          const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);  // 0 when m_ref = -inf
          l_run *= alpha;
#pragma unroll
          for (int n = 0; n < C::NPV; ++n) acc[n] *= alpha;
          m_ref = m_new;
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(p[s][i] - m_ref);  // exp2(-inf) = 0 for masked tokens
            p[s][i] = e;
            l_run += e;
          }
        }

        // 5. P' = p * (V scale | Lloyd-Max norm) as fp16 hi + lo.  A single
        // fp16 rounding of the weights costs up to 2^-11 relative per term,
        // which outputs formed by cancellation of large terms amplify.
        half8_t pbh[C::NB], pbl[C::NB];
#pragma unroll
        for (int nb = 0; nb < C::NB; ++nb) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float w = materialize(p[s][i] * io.vs[s][nb][i]);  // one value for hi and lo
              // masked tokens: p = 0 but the scale past the row end (or below
              // the window) may be any value
              if constexpr (MASKED) {
                const int tok = tb + 16 * s + 4 * g + i;
                w = (tok < t1 && (!WIN || tok >= lo_tok)) ? w : 0.0f;
              }
              const _Float16 wh = (_Float16)w;
              pbh[nb][4 * s + i] = wh;
              pbl[nb][4 * s + i] = (_Float16)(w - (float)wh);
            }
          }
        }

        // 6. prefetch the next tile's scales
        if constexpr (PREFETCH) issue_scales(tn, rn);

        // 7. PV: A = V^T through LDS transpose reads, B = P'^T
#pragma unroll
        for (int n = 0; n < C::NPV; ++n) {
          half8_t va;
          if constexpr (!K8V3) {
            const int off = (8 * g + ((lane >> 1) & 7)) * C::VROW + 16 * n + 8 * (lane & 1);
            const i32x2_t t = __builtin_amdgcn_ds_read_tr8_b64_v2i32((S8KV_LDS i32x2_t*)(vstage + off));
            va = i8x8_to_f16(__builtin_bit_cast(u32x2_t, t));
          } else {
            const int r0 = 8 * g + ((lane >> 2) & 3);
            const int colb = (16 * n + 4 * (lane & 3)) * 2;
            const i16x4_t lw =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((S8KV_LDS i16x4_t*)(vstage + r0 * C::VROW + colb));
            const i16x4_t hw =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((S8KV_LDS i16x4_t*)(vstage + (r0 + 4) * C::VROW + colb));
            const half4_t l4 = __builtin_bit_cast(half4_t, lw), h4 = __builtin_bit_cast(half4_t, hw);
            va = half8_t{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
          }
          const int nb = C::NB == 1 ? 0 : (16 * n) / 128;
          acc[n] = mfma16x16x32(va, pbh[nb], acc[n]);
          acc[n] = mfma16x16x32(va, pbl[nb], acc[n]);
        }
      };

      int tb = u0 + kTile * wave;
      const bool pre = pre_issued;  // (the first sub-split of the first segment only)
      pre_issued = false;
      if (tb < t1) {
        const uint32_t r0 = tile_in_block ? tile_row0(tb) : 0u;
        if (!pre || r0 != pre_r0) {  // (a tile issued from a plan that no longer applies is issued again)
          issue_kv(tb, r0);
          issue_scales(tb, r0);
        }
        if constexpr (WIN) {  // the row's first tile holds tokens below the window
          if (tb < lo_tok && tb + kTile * kDecWaves < t1) {
            process(tb, std::true_type{}, std::true_type{});
            tb += kTile * kDecWaves;
          }
        }
        while (tb + kTile * kDecWaves < t1) {  // a next tile exists, so this one is full
          process(tb, std::false_type{}, std::true_type{});
          S8KV_TRACE_STAMP_ONCE(kTrTile1);
          tb += kTile * kDecWaves;
        }
        if constexpr (FUSE) {
          if (app_seg && tb == padL - kTile) {  // the row's last tile: append its new token first
            // (the append kernel's arithmetic; runs while the tile's loads are in flight)
            const _Float16* nf = reinterpret_cast<const _Float16*>(smem + a.smem_new + C::NEW_F16K);
            float x[E], y[E];
#pragma unroll
            for (int e = 0; e < E; ++e) {  // lanes past a short row hold zeros (they enter the absmax)
              const bool on = lane < RowLayout<D>::ACTIVE;
              x[e] = on ? (float)nf[lane + 64 * e] : 0.0f;
              y[e] = on ? (float)nf[D + lane + 64 * e] : 0.0f;
            }
            fwht_row<D>(x, lane);
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = (float)(_Float16)materialize(x[e] * a.rot_norm);
            int qk[E];
            const float sk = rtn_row<D>(x, qk);
            uint32_t nrow = tile_in_block ? tile_row0(tb) + (uint32_t)(last - tb) : row_of(last);
            // (BIG: descriptors rebased to the new token's row, which then is row 0)
            rsrc_t kc_n = kc, ks_n = ks, vc_n = vc, vs_n = vs;
            if constexpr (BIG) {
              kc_n = window_rsrc(a.k_cache, a.kc_total, (uint64_t)nrow * D);
              ks_n = window_rsrc(a.k_scale, a.ks_total, (uint64_t)nrow * 4u);
              vc_n = window_rsrc(a.v_cache, a.vc_total, (uint64_t)nrow * (K8V3 ? C::WORDS * 4 : D));
              vs_n = window_rsrc(a.v_scale, a.vs_total, (uint64_t)nrow * (C::NB * 4u));
              nrow = 0;
            }
            char* nn = smem + a.smem_new;
            if (lane < RowLayout<D>::ACTIVE) {
#pragma unroll
              for (int e = 0; e < E; ++e) {
                bstore8((uint8_t)(int8_t)qk[e], kc_n, nrow * (uint32_t)D + lane + 64 * e);
                nn[C::NEW_I8K + lane + 64 * e] = (char)qk[e];
              }
            }
            if (lane == 0) {
              bstore32(__builtin_bit_cast(uint32_t, sk), ks_n, nrow * 4u);
              *reinterpret_cast<float*>(nn + C::NEW_KS) = sk;
            }
            if constexpr (!K8V3) {
              int qv[E];
              const float sv = rtn_row<D>(y, qv);
              if (lane < RowLayout<D>::ACTIVE) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                  bstore8((uint8_t)(int8_t)qv[e], vc_n, nrow * (uint32_t)D + lane + 64 * e);
                  nn[C::NEW_V + lane + 64 * e] = (char)qv[e];
                }
              }
              if (lane == 0) {
                bstore32(__builtin_bit_cast(uint32_t, sv), vs_n, nrow * 4u);
                *reinterpret_cast<float*>(nn + C::NEW_VS) = sv;
              }
            } else {  // 3-bit Lloyd-Max V: packed words and per-128 block norms
              float cb[8];
#pragma unroll
              for (int i = 0; i < 8; ++i) cb[i] = a.v_codebook[i];
              uint32_t w;
              float nv;
              lloydmax3_encode_row<D>(y, cb, lane, w, nv);
              if (lane < C::WORDS) {
                bstore32(w, vc_n, nrow * (uint32_t)(C::WORDS * 4) + lane * 4u);
                reinterpret_cast<uint32_t*>(nn + C::NEW_V)[lane] = w;
              }
              if (lane < C::NB) {
                bstore32(__builtin_bit_cast(uint32_t, nv), vs_n, nrow * (uint32_t)(C::NB * 4) + lane * 4u);
                reinterpret_cast<float*>(nn + C::NEW_VS)[lane] = nv;
              }
            }
          }
        }
        process(tb, std::true_type{}, std::false_type{});
      }
    }

    S8KV_TRACE_STAMP(kTrTilesEnd);
#ifdef S8KV_DECODE_TRACE
    tr_tok += (unsigned long long)(s1 - s0);
    tr_seg += 1;
    S8KV_TRACE_SET(kTrFlags, 1ull | ((unsigned long long)whole_row << 8));
#endif
    // ---- next segment: its set-up loads overlap this segment's merge ----
    int nb, npb, nL;
    if (reordered) {  // the reordered last segment is done: continue from the first
      nb = b_first;
      npb = pb_first;
      nL = L_first;
      reordered = false;
    } else {
      nb = b + 1;
      npb = pb + stream_len(a, L);
      nL = find_segment<WIN>(a, lens_lds, lo, hi, nb, npb);
      if (nb >= b_stop) nL = 0;
    }
    // (unconditional, from a valid row when there is no next segment: values
    // set on only one path would stay live across the tile loop)
    prefetch_segment(nL != 0 ? nb : b, nL != 0 ? max(lo, npb + a.ghost) - (npb + a.ghost) : 0);

    // ---- merge the waves of the workgroup in LDS ----
    {
    const int tid = opaque_int(threadIdx.x);
    const int lane = tid & 63;
    const int c = lane & 15;
    const int g = lane >> 4;
    const float l_tot = sum_x32(sum_x16(l_run));
    __syncthreads();  // every wave is done with its V staging and the staged block ids
    float* mrg = reinterpret_cast<float*>(smem);
    const int wstride = G * D + 32;
    float* w_acc = mrg + wave * wstride;  // [G heads][D], then m[16], l[16]
    if (c < G) {
#pragma unroll
      for (int n = 0; n < C::NPV; ++n) {
#pragma unroll
        for (int r = 0; r < 4; ++r) w_acc[c * D + 16 * n + 4 * g + r] = acc[n][r];
      }
      if (g == 0) {
        w_acc[G * D + c] = m_ref;  // l and acc are relative to 2^m_ref
        w_acc[G * D + 16 + c] = l_tot;
      }
    }
    __syncthreads();
    // bt_lds is free: every wave left its tile loop (the last segment stages
    // nothing, so the workgroup's end does not wait for the prefetch's loads)
    if (nL != 0) store_prefetched_bt();
    const int64_t slot = ((int64_t)h * a.slots + (j + b)) * G;  // (row, slice) -> unique slot j + b
    for (int i = tid; i < G * D; i += 64 * kDecWaves) {
      const int cc = i / D, d = i - cc * D;
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, mrg[w * wstride + G * D + cc]);
      float num = 0.0f, den = 0.0f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float* wa = mrg + w * wstride;
        const float mw = wa[G * D + cc];
        const float f = (mw == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
        num += f * wa[cc * D + d];
        den += f * wa[G * D + 16 + cc];
      }
      if (whole_row) {
        a.out[((int64_t)b * a.num_q_heads + h * G + cc) * D + d] = (_Float16)(den > 0.0f ? num / den : 0.0f);
      } else {
        store_agent(&a.ws_acc[(slot + cc) * D + d], num);
        if (d == 0) {
          store_agent(&a.ws_ml[(slot + cc) * 2], M);
          store_agent(&a.ws_ml[(slot + cc) * 2 + 1], den);
        }
      }
    }
    if (!whole_row) {
      // ---- arrival: the segment completing the row combines its partials ----
      __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have reached the coherence point
      __syncthreads();
      __shared__ int completes_row;
      if (tid == 0)
        completes_row = arrive(a.ws_cnt + (int64_t)h * a.batch + b, a.tag, (uint32_t)(s1 - s0) >> 5,
                               (uint32_t)padL >> 5);
      __syncthreads();
#ifdef S8KV_DECODE_TRACE
      if (completes_row) S8KV_TRACE_SET(kTrFlags, trace_lds[kTrFlags] | (1ull << 9));
#endif
      if (completes_row) {
        // slices jf..jl hold the row's segments; their partials are at slots j + b
        // (recomputed here from opaque copies of its inputs, so that no part of
        // it is hoisted from the prologue and kept live across the tile loop)
        int jf, jl;
        if (adapt) {  // the largest columns whose bounds are at or before the row's first and last tokens
          const int32_t* bd = a.plan + plan_adapt_off(a.plan_wmax) + kAdBounds;
          const int ln = opaque_int(threadIdx.x) & 63, W = a.wg_per_head;
          int nf = 0, nl = 0;
          for (int c0 = 0; c0 < W; c0 += 256) {  // four loads in flight
            int v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = c0 + 64 * u + ln < W ? bd[c0 + 64 * u + ln] : 0x7FFFFFFF;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              nf += __builtin_popcountll(__builtin_amdgcn_ballot_w64(v[u] <= rs));
              nl += __builtin_popcountll(__builtin_amdgcn_ballot_w64(v[u] <= rs + padL - 1));
            }
          }
          jf = nf - 1;
          jl = nl - 1;
        } else {
          const SliceLayout sm = slice_layout(opaque_int(total), opaque_int(a.wg_per_head),
                                              opaque_int(a.slot_classes), opaque_int(a.slot_skew),
                                              opaque_int(threadIdx.x) & 63);
          jf = slice_of(sm, rs);
          jl = slice_of(sm, rs + padL - 1);
        }
        for (int i = tid; i < G * D; i += 64 * kDecWaves) {
          const int cc = i / D, d = i - cc * D;
          float M = kNegInf, num = 0.0f, den = 0.0f;
          for (int j0 = jf; j0 <= jl; j0 += 4) {  // four partials' loads in flight at a time
            float ms[4], ls[4], xs[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int jj = min(j0 + u, jl);
              const int64_t pi = ((int64_t)h * a.slots + jj + b) * G + cc;
              ms[u] = j0 + u <= jl ? load_agent(&a.ws_ml[pi * 2]) : kNegInf;
              ls[u] = load_agent(&a.ws_ml[pi * 2 + 1]);
              xs[u] = load_agent(&a.ws_acc[pi * D + d]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              if (ms[u] == kNegInf) continue;  // past jl, or a segment that saw no token
              if (ms[u] > M) {
                const float f = __builtin_amdgcn_exp2f(M - ms[u]);  // 0 while M = -inf
                num *= f;
                den *= f;
                M = ms[u];
              }
              const float f = __builtin_amdgcn_exp2f(ms[u] - M);
              num += f * xs[u];
              den += f * ls[u];
            }
          }
          a.out[((int64_t)b * a.num_q_heads + h * G + cc) * D + d] = (_Float16)(den > 0.0f ? num / den : 0.0f);
        }
      }
    }
    }
    if (nL == 0) break;
    b = nb;
    pb = npb;
    L = nL;
  }
  if (adapt) {  // (workgroup-uniform) the end: when the last wave is done
    __syncthreads();
    record_times();
  }
#ifdef S8KV_DECODE_TRACE
  S8KV_TRACE_STAMP(kTrExit);
  S8KV_TRACE_SET(kTrWork, tr_tok | (tr_seg << 32));
  S8KV_TRACE_SET(kTrHwId, (unsigned long long)__smid());
  __syncthreads();
  if (a.trace != nullptr && threadIdx.x < kTraceWords)
    a.trace[(int64_t)blockIdx.x * kTraceWords + threadIdx.x] = trace_lds[threadIdx.x];
#endif
}

// ---- adaptive slice bounds ----
// Wave sums and prefix sums of floats (ds_swizzle / DPP-free shuffles; the
// bounds kernel is one wave and runs once per step).
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_incl_scan_f(float v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  return v;
}
// slice_start for a per-lane column j (0 <= j < W).
__device__ __forceinline__ int slice_start_lane(const SliceLayout& s, int j) {
  int r = 0;
#pragma unroll
  for (int c = 0; c < kMaxResidentPerCU; ++c) {
    const int f0 = __builtin_amdgcn_readlane(s.f0, c), f1 = __builtin_amdgcn_readlane(s.f1, c);
    if (f0 <= j && j < f1) r = __builtin_amdgcn_readlane(s.start, c) + (j - f0) * __builtin_amdgcn_readlane(s.sz, c);
  }
  return r;
}

// Slice bounds of an adaptive plan, bd[0..W] (one workgroup).  When the plan
// buffer holds this geometry's bounds, its stream total moved by at most a
// sixteenth, and every workgroup of the last launch that read the plan
// recorded its times under the plan's epoch, each column's share of the
// stream moves a fraction kAdaptGain (S8KV_DECODE_ADAPT_GAIN overrides it)
// of the way from its last share towards the share its measured rate earns
// -- slice length over finish time, the end stamp minus the launch's
// earliest start, summed over the KV heads -- changing by at most kAdaptStep
// of itself and staying at or above kAdaptFloor of an even share (where a
// column the formula left past the stream's end starts from).  At the fixed
// point every column finishes at the same time.  Otherwise the bounds are
// the formula's (those of the unplanned slicing).  Bounds are multiples of
// 32 (the last one is the stream total), non-decreasing, with bd[0] = 0; the
// epoch advances by one.
constexpr int kAdaptMaxCols = 2048;
constexpr float kAdaptGain = 0.25f;
constexpr float kAdaptStep = 0.25f;
constexpr float kAdaptFloor = 0.25f;
constexpr int kAdaptMinTokens = 128;  // stream tokens per column below which the formula is kept
template <bool WIN>
__global__ __launch_bounds__(64 * kDecWaves) void decode_bounds_kernel(DecodeArgs a) {
  constexpr int NT = 64 * kDecWaves;
  __shared__ int lens_lds[kLensLds];
  __shared__ float len_lds[kAdaptMaxCols];
  __shared__ float rate_lds[kAdaptMaxCols];
  __shared__ int red_i[2 * kDecWaves];
  __shared__ float red_f[2 * kDecWaves];
  __shared__ int nb_lds[kAdaptMaxCols + 1];  // the new bounds before spacing
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int i = tid; i < min(a.batch, kLensLds); i += NT) lens_lds[i] = a.context_lens[i];
  __syncthreads();
  int32_t* ad = a.plan_out + plan_adapt_off(a.plan_wmax);
  int32_t* bd = ad + kAdBounds;
  const int32_t* fb = a.plan_out + plan_fb_off(a.plan_wmax);
  const int W = a.wg_per_head, Hkv = a.num_kv_heads;
  const int total = stream_total<WIN>(a, lens_lds, lane);
  const bool known = ad[kAdMagic] == kAdaptMagic;
  const int epoch = ad[kAdEpoch];
  const int64_t old_total = ad[kAdTotal];
  bool ok = known && ad[kAdWg] == W && ad[kAdHkv] == Hkv && ad[kAdBatch] == a.batch && W <= kAdaptMaxCols &&
            W <= a.plan_wmax && (int64_t)total >= (int64_t)kAdaptMinTokens * W && old_total > 0 &&
            16 * (int64_t)abs(total - (int)old_total) <= old_total && bd[0] == 0 && bd[W] == (int)old_total;
  // every entry is the last launch's; its earliest start, relative to entry (0, 0)'s
  const uint32_t ref = ok ? (uint32_t)fb[1] : 0u;
  {
    bool mine = true;
    int dmin = 0;
    if (ok) {
      for (int i = tid; i < W * Hkv; i += NT) {
        const int hh = i / W, jj = i - hh * W;
        const int32_t* f = fb + ((int64_t)hh * a.plan_wmax + jj) * kFbWords;
        mine = mine && f[0] == epoch;
        dmin = min(dmin, (int)((uint32_t)f[1] - ref));
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) dmin = min(dmin, __shfl_xor(dmin, off, 64));
    if (lane == 0) {
      red_i[wave] = __builtin_amdgcn_ballot_w64(!mine) == 0;
      red_i[kDecWaves + wave] = dmin;
    }
  }
  __syncthreads();
  int dmin = 0;
#pragma unroll
  for (int w = 0; w < kDecWaves; ++w) {
    ok = ok && red_i[w] != 0;
    dmin = min(dmin, red_i[kDecWaves + w]);
  }
  // each column's last slice length and rate
  {
    bool sane = true;
    float sum_len = 0.0f, sum_rate = 0.0f;
    if (ok) {
      for (int jj = tid; jj < W; jj += NT) {
        const int lo = bd[jj], hi = bd[jj + 1];
        float t = 0.0f;
        for (int hh = 0; hh < Hkv; ++hh) {
          const int32_t* f = fb + ((int64_t)hh * a.plan_wmax + jj) * kFbWords;
          t += (float)((int)((uint32_t)f[2] - ref) - dmin);
        }
        sane = sane && hi >= lo && (hi == lo || t > 0.0f);
        const float len = (float)(hi - lo);
        const float rate = hi > lo ? len / t : 0.0f;  // a column past the stream's end: rate 0 (it gets the floor share)
        len_lds[jj] = len;
        rate_lds[jj] = rate;
        sum_len += len;
        sum_rate += rate;
      }
    }
    sum_len = wave_sum_f(sum_len);
    sum_rate = wave_sum_f(sum_rate);
    __syncthreads();  // (red_i read by every thread above)
    if (lane == 0) {
      red_i[wave] = __builtin_amdgcn_ballot_w64(!sane) == 0;
      red_f[wave] = sum_len;
      red_f[kDecWaves + wave] = sum_rate;
    }
  }
  __syncthreads();
  float sum_len = 0.0f, sum_rate = 0.0f;
#pragma unroll
  for (int w = 0; w < kDecWaves; ++w) {  // (fixed order)
    ok = ok && red_i[w] != 0;
    sum_len += red_f[w];
    sum_rate += red_f[kDecWaves + w];
  }
  ok = ok && sum_len > 0.0f && sum_rate > 0.0f;
  if (wave != 0) return;
  if (ok) {
    // the new shares (in len_lds), then their prefix sums scaled to the stream
    const float floor_share = kAdaptFloor / (float)W;
    float sum_new = 0.0f;
    for (int c0 = 0; c0 < W; c0 += 64) {
      const int jj = c0 + lane;
      float f = 0.0f;
      if (jj < W) {
        const float fo = len_lds[jj] / sum_len, ft = rate_lds[jj] / sum_rate;
        f = fo + a.adapt_gain * (ft - fo);
        f = fminf(fmaxf(f, fo * (1.0f - kAdaptStep)), fo * (1.0f + kAdaptStep));
        f = fmaxf(f, floor_share);
        len_lds[jj] = f;
      }
      sum_new += wave_sum_f(f);
    }
    const float units = (float)(total >> 5) / sum_new;
    float carry = 0.0f;
    for (int c0 = 0; c0 < W; c0 += 64) {
      const int jj = c0 + lane;
      const float incl = wave_incl_scan_f(jj < W ? len_lds[jj] : 0.0f, lane) + carry;
      if (jj + 1 < W) {
        const int nb = min(total, 32 * (int)rintf(incl * units));
        nb_lds[jj + 1] = nb;
      }
      carry = __shfl(incl, 63, 64);
    }
    // every slice inside the stream holds at least a tile: bd[j] = max over
    // i <= j of (b[i] + 32 (j - i)), capped at the total (an empty slice in
    // the middle of a row would hold no segment of it, and the row's
    // combine would read that column's slot, which no launch wrote)
    if (lane == 0) nb_lds[0] = 0;
    int run = 0;  // max over the earlier chunks of b[i] - 32 i
    for (int c0 = 0; c0 < W; c0 += 64) {
      const int jj = c0 + lane;
      int v = jj < W ? nb_lds[jj] - kTile * jj : -0x7FFFFFFF;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(v, off, 64);
        if (lane >= off) v = max(v, t);
      }
      v = max(v, run);
      if (jj > 0 && jj < W) bd[jj] = min(total, v + kTile * jj);
      run = __shfl(v, 63, 64);
    }
  } else {
    const SliceLayout sl = slice_layout(total, W, a.slot_classes, a.slot_skew, lane);
    for (int c0 = 1; c0 < W; c0 += 64) {
      const int jj = c0 + lane;
      if (jj < W) bd[jj] = min(total, slice_start_lane(sl, jj));
    }
  }
  if (lane == 0) {
    bd[0] = 0;
    bd[W] = total;
    ad[kAdMagic] = kAdaptMagic;
    ad[kAdWg] = W;
    ad[kAdHkv] = Hkv;
    ad[kAdBatch] = a.batch;
    ad[kAdEpoch] = known ? epoch + 1 : 1;
    ad[kAdTotal] = total;
  }
}

// The step's slice plan: one wave per workgroup column j, the decode
// prologue's arithmetic on the same lengths (locate_slice), plus the storage
// row (KV head 0) of each wave's first tile in the segment processed first --
// tile s0 + 32 w of the segment's first sub-split, when it exists and the
// block size keeps a tile inside one block.  Block 0 also writes the header.
template <bool WIN, bool ADAPT = false>
__global__ __launch_bounds__(64 * kDecWaves) void decode_plan_kernel(DecodeArgs a) {
  __shared__ int lens_lds[kLensLds];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = blockIdx.x * kDecWaves + wave;
  int32_t* plan = a.plan_out;
  for (int i = tid; i < min(a.batch, kLensLds); i += 64 * kDecWaves) lens_lds[i] = a.context_lens[i];
  if (blockIdx.x == 0 && tid < kPlanHeader && tid != kPlanLensWord)
    plan[tid] = tid == kPlanAdaptWord ? (ADAPT ? 1 : 0) : plan_header_word(a, tid);
  __syncthreads();
  if (blockIdx.x == 0 && wave == 0) {
    const uint32_t cs = lens_checksum(a, lens_lds, lane);
    if (lane == 0) plan[kPlanLensWord] = (int32_t)cs;
  }
  if (j >= a.wg_per_head) return;
  SliceLoc s;
  bool found;
  if constexpr (ADAPT) {  // the slice bounds decode_bounds_kernel wrote for this step
    const int32_t* bd = plan + plan_adapt_off(a.plan_wmax) + kAdBounds;
    s.total = stream_total<WIN>(a, lens_lds, lane);
    s.lo = min(bd[j], s.total);
    s.hi = min(bd[j + 1], s.total);
    found = slice_segments<WIN>(a, lens_lds, lane, s);
  } else {
    found = locate_slice<WIN>(a, lens_lds, j, lane, s);
  }
  if (!found) {  // no segment: the launch's workgroup j returns at once
    if (s.lo >= s.total) s.lo = s.hi = s.total;
    s.L = 0;
    s.b = s.pb = s.b_first = s.pb_first = s.L_first = s.reordered = 0;
    s.b_stop = a.batch;
  }
  uint32_t r0 = kNoTile;
  if (s.L > 0 && a.bs_log2 >= 5 && lane < kDecWaves) {
    const int rs = s.pb + a.ghost;
    const int s0 = max(s.lo, rs) - rs;
    const int s1 = min(s.hi, rs + padded32(s.L)) - rs;
    const int t1 = min(min(s1, s0 + kSubTokens), s.L);
    const int al = WIN ? win_base(a, lens_at(a, lens_lds, s.b)) : 0;
    const int tb = s0 + kTile * lane + al;
    if (s0 + kTile * lane < t1) {
      const uint32_t blk = (uint32_t)a.block_table[(int64_t)s.b * a.bt_stride + (tb >> a.bs_log2)];
      r0 = ((blk * (uint32_t)a.num_kv_heads) << a.bs_log2) + ((uint32_t)tb & ((1u << a.bs_log2) - 1u));
    }
  }
  const int w0 = __builtin_amdgcn_readlane((int)r0, 0), w1 = __builtin_amdgcn_readlane((int)r0, 1);
  const int w2 = __builtin_amdgcn_readlane((int)r0, 2), w3 = __builtin_amdgcn_readlane((int)r0, 3);
  if (lane < kPlanEntry) {
    int v = 0;
    switch (lane) {
      case kPwTotal: v = s.total; break;
      case kPwLo: v = s.lo; break;
      case kPwHi: v = s.hi; break;
      case kPwB: v = s.b; break;
      case kPwPb: v = s.pb; break;
      case kPwL: v = s.L; break;
      case kPwBFirst: v = s.b_first; break;
      case kPwPbFirst: v = s.pb_first; break;
      case kPwLFirst: v = s.L_first; break;
      case kPwBStop: v = s.b_stop; break;
      case kPwReordered: v = s.reordered; break;
      case kPwTile0: v = w0; break;
      case kPwTile0 + 1: v = w1; break;
      case kPwTile0 + 2: v = w2; break;
      case kPwTile0 + 3: v = w3; break;
      default: v = 0;
    }
    plan[kPlanHeader + (int64_t)j * kPlanEntry + lane] = v;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Kernel timing (diagnostics): while enabled, every decode call launches its
// kernel with HIP events stamped with the kernel's start and end time
// (hipExtLaunchKernelGGL).  Calls under graph capture are not timed.
#ifdef S8KV_DECODE_TRACE
// Trace buffer of the diagnostics build: consecutive launches take
// consecutive slots of the caller's buffer (modulo its slot count), each
// `stride` words; launches that need more than a slot are not traced.
struct TraceState {
  unsigned long long* buf = nullptr;
  int64_t stride = 0, slots = 0, next = 0;
};
static TraceState g_trace;
static unsigned long long* trace_slot(int64_t words) {
  if (g_trace.buf == nullptr || g_trace.slots <= 0 || words > g_trace.stride) return nullptr;
  return g_trace.buf + (g_trace.next++ % g_trace.slots) * g_trace.stride;
}
#endif

struct TimingState {
  bool on = false;
  std::vector<std::array<hipEvent_t, 2>> events;
  size_t used = 0;
};
static TimingState g_timing;

static hipEvent_t* timing_slot(hipStream_t stream) {
  if (!g_timing.on) return nullptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  if (g_timing.used == g_timing.events.size()) {
    std::array<hipEvent_t, 2> e{};
    for (auto& x : e)
      if (hipEventCreate(&x) != hipSuccess) return nullptr;
    g_timing.events.push_back(e);
  }
  return g_timing.events[g_timing.used++].data();
}


// Workgroups per KV head: about the number the GPU keeps resident, split
// evenly over the heads.  S8KV_DECODE_WG_PER_HEAD overrides it (clamped to
// the bound the workspace is sized for) to exercise other slicings.
static int max_wg_per_head(int num_kv_heads) {
  const int w = device_cus() * kMaxResidentPerCU / num_kv_heads;
  return w > 0 ? w : 1;
}
static int plan_wg_per_head(int num_kv_heads, int resident_per_cu) {
  const int cap = max_wg_per_head(num_kv_heads);
  int w = device_cus() * resident_per_cu / num_kv_heads;
  if (const char* env = getenv("S8KV_DECODE_WG_PER_HEAD")) {
    const int v = atoi(env);
    if (v > 0) w = v;
  }
  return w < 1 ? 1 : (w > cap ? cap : w);
}

template <int D, bool K8V3, bool FUSE, bool WIN, bool BIG>
static int launch_decode_impl(DecodeArgs& a, hipStream_t stream) {
  using C = DecCfg<D, K8V3>;
  constexpr int kNewBytes = FUSE ? C::NEW_BYTES : 0;  // fused append: the new token's rows
  const auto smem_main_for = [](int group) {  // V staging + rotated q, or the cross-wave merge
    const int merge = kDecWaves * (group * D + 32) * 4;
    const int stage_q = C::SMEM_Q + 4 * group * D;
    return ((stage_q > merge ? stage_q : merge) + 15) / 16 * 16;
  };
  a.smem_main = smem_main_for(a.group);
  a.smem_new = a.smem_main + (kMaxSubBlocks + kLensLds) * 4;
  const int smem = a.smem_new + kNewBytes;
  // Resident workgroups per CU at this LDS size (depends on the GQA group),
  // queried once per group size.
  static int resident_by_group[17] = {};
  static bool lds_raised = false;
  if (!lds_raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_kernel<D, K8V3, FUSE, WIN, BIG>),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            smem_main_for(16) + (kMaxSubBlocks + kLensLds) * 4 + kNewBytes) != hipSuccess) {
      set_error("s8kv_decode: cannot raise the dynamic LDS limit");
      return S8KV_ERR_LAUNCH;
    }
    lds_raised = true;
  }
  int& resident = resident_by_group[a.group];
  if (resident == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<D, K8V3, FUSE, WIN, BIG>, 64 * kDecWaves, smem) != hipSuccess ||
        n <= 0)
      n = 2;
    resident = n < kMaxResidentPerCU ? n : kMaxResidentPerCU;
  }
  a.wg_per_head = plan_wg_per_head(a.num_kv_heads, resident);
  a.ghost = kGhostTokens;
  a.slot_classes = resident;
  if (const char* env = getenv("S8KV_DECODE_CLASSES")) {  // residency classes the slices are weighted over
    const int v = atoi(env);
    a.slot_classes = v < 1 ? 1 : (v > kMaxResidentPerCU ? kMaxResidentPerCU : v);
  }
  a.slot_skew = kSlotSkewPermille;
  if (const char* env = getenv("S8KV_DECODE_SLOT_SKEW")) a.slot_skew = atoi(env);
  if (const char* env = getenv("S8KV_DECODE_GHOST")) {
    const int g = atoi(env);
    a.ghost = (g < 0 ? 0 : (g > (1 << 16) ? (1 << 16) : g) + 31) / 32 * 32;
  }
  // stream positions are int32: every row's padded length plus its ghost
  // tokens, summed over the batch, must stay below 2^31
  if ((int64_t)a.batch * ((int64_t)a.max_context_len + 31 + a.ghost) >= (int64_t(1) << 31)) {
    set_error("s8kv_decode: batch * (max_context_len + %d) too large", a.ghost + 31);
    return S8KV_ERR_UNSUPPORTED;
  }
  a.slots = a.batch + a.wg_per_head;
  if (a.plan_out != nullptr) {  // s8kv_decode_plan: the slice plan of this launch geometry
    const dim3 pgrid((a.wg_per_head + kDecWaves - 1) / kDecWaves);
    if (a.plan_adapt) {
      if (a.wg_per_head > kAdaptMaxCols) {
        set_error("s8kv_decode_plan_adaptive: %d workgroups per KV head > %d", a.wg_per_head, kAdaptMaxCols);
        return S8KV_ERR_UNSUPPORTED;
      }
      a.adapt_gain = kAdaptGain;
      if (const char* env = getenv("S8KV_DECODE_ADAPT_GAIN")) {
        const float g = (float)atof(env);
        a.adapt_gain = g < 0.0f ? 0.0f : (g > 1.0f ? 1.0f : g);
      }
      hipLaunchKernelGGL((decode_bounds_kernel<WIN>), dim3(1), dim3(64 * kDecWaves), 0, stream, a);
      hipLaunchKernelGGL((decode_plan_kernel<WIN, true>), pgrid, dim3(64 * kDecWaves), 0, stream, a);
    } else {
      hipLaunchKernelGGL((decode_plan_kernel<WIN>), pgrid, dim3(64 * kDecWaves), 0, stream, a);
    }
    return check_launch(a.plan_adapt ? "s8kv_decode_plan_adaptive" : "s8kv_decode_plan");
  }
  const dim3 grid(a.wg_per_head * a.num_kv_heads);
#ifdef S8KV_DECODE_TRACE
  a.trace = trace_slot((int64_t)grid.x * kTraceWords);
#endif
  hipEvent_t* ev = a.untimed ? nullptr : timing_slot(stream);
  if (ev) {  // events stamped with the kernel's own start and end times
    hipExtLaunchKernelGGL((decode_kernel<D, K8V3, FUSE, WIN, BIG>), grid, dim3(64 * kDecWaves), smem, stream, ev[0], ev[1], 0, a);
  } else {
    hipLaunchKernelGGL((decode_kernel<D, K8V3, FUSE, WIN, BIG>), grid, dim3(64 * kDecWaves), smem, stream, a);
  }
  return check_launch("s8kv_decode");
}
template <int D, bool K8V3, bool FUSE, bool WIN = false>
static int launch_decode(DecodeArgs& a, hipStream_t stream) {
  return a.big ? launch_decode_impl<D, K8V3, FUSE, WIN, true>(a, stream)
               : launch_decode_impl<D, K8V3, FUSE, WIN, false>(a, stream);
}

// Workspace: (max, sum) and unnormalised output partials of every (q head,
// slot), then the arrival counters of every (KV head, row).  The partials'
// size is a multiple of 8 bytes (head_dim + 2 is even), so the counters are
// 8-byte aligned when the workspace is.
static int64_t partial_count(int batch, int num_q_heads, int num_kv_heads) {
  return (int64_t)num_q_heads * (batch + max_wg_per_head(num_kv_heads));  // (q head, slot) pairs
}
static int64_t workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int head_dim) {
  return partial_count(batch, num_q_heads, num_kv_heads) * (head_dim + 2) * 4 + (int64_t)num_kv_heads * batch * 8;
}
// Slice plan: header + one entry per workgroup column, for the largest grid
// a launch of this geometry may use.
// Adaptive plans also hold the slice bounds and one feedback entry per
// (KV head, column).
static int64_t plan_bytes_for(int num_kv_heads) {
  const int w = max_wg_per_head(num_kv_heads);
  return (plan_fb_off(w) + (int64_t)kFbWords * num_kv_heads * w) * 4;
}


static int decode_common(DecodeArgs& a, bool k8v3, bool fuse, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                         int64_t num_blocks, int block_size, int max_context_len, float scale, void* workspace,
                         int64_t workspace_bytes_given, void* stream) {
  S8KV_REQUIRE(batch >= 0, S8KV_ERR_INVALID, "decode: batch < 0");
  if (batch == 0) return S8KV_OK;
  S8KV_REQUIRE(batch <= 65535, S8KV_ERR_UNSUPPORTED, "decode: batch %d > 65535", batch);
  S8KV_REQUIRE(num_kv_heads > 0 && num_q_heads > 0 && num_q_heads % num_kv_heads == 0, S8KV_ERR_INVALID,
               "decode: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads, num_kv_heads);
  S8KV_REQUIRE(num_q_heads / num_kv_heads <= 16, S8KV_ERR_UNSUPPORTED, "decode: more than 16 q heads per kv head");
  S8KV_REQUIRE(head_dim_ok(head_dim), S8KV_ERR_UNSUPPORTED, "decode: head_dim %d not in {32,64,128,256}", head_dim);
  S8KV_REQUIRE(!k8v3 || head_dim == 128 || head_dim == 256, S8KV_ERR_UNSUPPORTED,
               "decode_k8v3: head_dim %d not in {128, 256}", head_dim);
  S8KV_REQUIRE(is_pow2(block_size) && block_size >= 4, S8KV_ERR_UNSUPPORTED,
               "decode: block_size %d must be a power of two >= 4", block_size);
  S8KV_REQUIRE(num_blocks > 0, S8KV_ERR_INVALID, "decode: num_blocks must be > 0");
  S8KV_REQUIRE(max_context_len >= 0, S8KV_ERR_INVALID, "decode: max_context_len < 0");
  S8KV_REQUIRE(max_context_len < (1 << 28), S8KV_ERR_UNSUPPORTED, "decode: max_context_len %d >= 2^28",
               max_context_len);
  S8KV_REQUIRE((int64_t)batch * (max_context_len + 31) < (int64_t(1) << 31), S8KV_ERR_UNSUPPORTED,
               "decode: batch * max_context_len too large");
  const bool plan_only = a.plan_out != nullptr;  // s8kv_decode_plan: reads lengths and block table only
  S8KV_REQUIRE(a.block_table && a.context_lens, S8KV_ERR_INVALID, "decode: null block table or context lengths");
  S8KV_REQUIRE(plan_only || (a.q && a.k_cache && a.k_scale && a.v_cache && a.v_scale && a.out), S8KV_ERR_INVALID,
               "decode: null pointer argument");
  S8KV_REQUIRE(plan_only || !fuse || (a.k_new && a.v_new), S8KV_ERR_INVALID, "decode_append: null k_new / v_new");
  const int64_t rows = num_blocks * num_kv_heads * block_size;
  S8KV_REQUIRE(fits_u32(rows), S8KV_ERR_UNSUPPORTED, "decode: more than 2^32 cache rows per layer");
  // a tensor past 4 GiB: tiles through descriptors rebased per tile, which
  // needs tiles inside one block
  a.big = !fits_u32(rows * head_dim);
  S8KV_REQUIRE(!a.big || block_size >= 32, S8KV_ERR_UNSUPPORTED,
               "decode: a per-layer cache past 4 GiB needs block_size >= 32 (got %d)", block_size);
  a.batch = batch;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.kc_total = (uint64_t)(rows * head_dim);
  a.ks_total = (uint64_t)(rows * 4);
  a.vc_total = (uint64_t)(k8v3 ? rows * (head_dim / 32 * 3) * 4 : rows * head_dim);
  a.vs_total = (uint64_t)(k8v3 ? rows * (head_dim / 128) * 4 : rows * 4);
  a.kc_bytes = cap_u32(a.kc_total);  // (BIG: unused by the tiles)
  a.ks_bytes = cap_u32(a.ks_total);
  a.vc_bytes = cap_u32(a.vc_total);
  a.vs_bytes = cap_u32(a.vs_total);
  a.bs_log2 = log2i(block_size);
  a.max_context_len = max_context_len;
  a.plan_wmax = max_wg_per_head(num_kv_heads);
  a.qscale = (float)((double)scale * 1.4426950408889634 / __builtin_sqrt((double)head_dim));
  a.rot_norm = (float)(1.0 / __builtin_sqrt((double)head_dim));
  if (plan_only) {
    S8KV_REQUIRE(workspace_bytes_given >= plan_bytes_for(num_kv_heads) && (uintptr_t)a.plan_out % 4 == 0,
                 S8KV_ERR_INVALID, "decode_plan: a plan of %lld bytes (4-byte aligned) is needed, %lld given",
                 (long long)plan_bytes_for(num_kv_heads), (long long)workspace_bytes_given);
  } else {
    const int64_t need = workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim);
    S8KV_REQUIRE(workspace != nullptr && workspace_bytes_given >= need, S8KV_ERR_WORKSPACE,
                 "decode: workspace of %lld bytes needed, %lld given", (long long)need,
                 (long long)workspace_bytes_given);
    S8KV_REQUIRE((uintptr_t)workspace % 8 == 0, S8KV_ERR_WORKSPACE, "decode: workspace not 8-byte aligned");
    const int64_t partials = partial_count(batch, num_q_heads, num_kv_heads);
    a.ws_ml = reinterpret_cast<float*>(workspace);
    a.ws_acc = a.ws_ml + partials * 2;
    a.ws_cnt = reinterpret_cast<unsigned long long*>(a.ws_acc + partials * head_dim);
    a.tag = next_launch_tag();
  }
  hipStream_t s = (hipStream_t)stream;
  if (a.window > 0) {  // sliding window (no fused append)
    switch (head_dim) {
      case 32: return k8v3 ? S8KV_ERR_UNSUPPORTED : launch_decode<32, false, false, true>(a, s);
      case 64: return k8v3 ? S8KV_ERR_UNSUPPORTED : launch_decode<64, false, false, true>(a, s);
      case 128: return k8v3 ? launch_decode<128, true, false, true>(a, s) : launch_decode<128, false, false, true>(a, s);
      case 256: return k8v3 ? launch_decode<256, true, false, true>(a, s) : launch_decode<256, false, false, true>(a, s);
    }
    return S8KV_ERR_UNSUPPORTED;
  }
  if (fuse) {
    if (k8v3) {
      switch (head_dim) {
        case 128: return launch_decode<128, true, true>(a, s);
        case 256: return launch_decode<256, true, true>(a, s);
      }
      return S8KV_ERR_UNSUPPORTED;
    }
    switch (head_dim) {
      case 32: return launch_decode<32, false, true>(a, s);
      case 64: return launch_decode<64, false, true>(a, s);
      case 128: return launch_decode<128, false, true>(a, s);
      case 256: return launch_decode<256, false, true>(a, s);
    }
    return S8KV_ERR_UNSUPPORTED;
  }
  switch (head_dim) {
    case 32: return k8v3 ? S8KV_ERR_UNSUPPORTED : launch_decode<32, false, false>(a, s);
    case 64: return k8v3 ? S8KV_ERR_UNSUPPORTED : launch_decode<64, false, false>(a, s);
    case 128: return k8v3 ? launch_decode<128, true, false>(a, s) : launch_decode<128, false, false>(a, s);
    case 256: return k8v3 ? launch_decode<256, true, false>(a, s) : launch_decode<256, false, false>(a, s);
  }
  return S8KV_ERR_UNSUPPORTED;
}

}  // namespace s8kv

// Scratch of the allocation-free entry point (s8kv_decode_append_int8_noalloc):
// the decode workspace (split-row partials and arrival counters) in a
// file-scope device array.  Each GPU the library runs on holds its own copy
// until the process ends.
constexpr int64_t kScratchBytes = S8KV_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace s8kv {

constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchDevices] = {};

// Device address of the current device's copy of `scratch`, looked up once per
// device with that device current.  In host code the array's name is only a
// stand-in for the symbol: kernels and copies must be given this address.
static int scratch_for_current_device(void** out) {
  int dev = -1;
  S8KV_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kScratchDevices, S8KV_ERR_LAUNCH,
               "decode_append_int8_noalloc: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    S8KV_REQUIRE(e == hipSuccess && p != nullptr, S8KV_ERR_LAUNCH,
                 "decode_append_int8_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                 hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return S8KV_OK;
}

}  // namespace s8kv

using namespace s8kv;

#ifdef S8KV_DECODE_TRACE
// Diagnostics build only: route the records of the next decode launches to a
// device buffer of `slots` x `stride` 64-bit words (null: stop tracing).
extern "C" int s8kv_decode_trace_set(void* buffer, int64_t stride_words, int64_t slots) {
  g_trace.buf = static_cast<unsigned long long*>(buffer);
  g_trace.stride = stride_words;
  g_trace.slots = slots;
  g_trace.next = 0;
  return S8KV_OK;
}
#endif

extern "C" int s8kv_timing_begin(void) {
  g_timing.on = true;
  g_timing.used = 0;
  return S8KV_OK;
}

extern "C" int s8kv_timing_end(int* launches, double* decode_ms, double* merge_ms) {
  g_timing.on = false;
  double dk = 0.0;
  for (size_t i = 0; i < g_timing.used; ++i) {
    auto& e = g_timing.events[i];
    if (hipEventSynchronize(e[1]) != hipSuccess) {
      set_error("s8kv_timing_end: event synchronize failed");
      return S8KV_ERR_LAUNCH;
    }
    float a = 0.f;
    hipEventElapsedTime(&a, e[0], e[1]);
    dk += a;
  }
  if (launches) *launches = (int)g_timing.used;
  if (decode_ms) *decode_ms = dk;
  if (merge_ms) *merge_ms = 0.0;  // the merge runs inside the decode kernel
  g_timing.used = 0;
  return S8KV_OK;
}

extern "C" int64_t s8kv_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                              int max_context_len) {
  (void)max_context_len;
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  return workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim);
}

extern "C" int s8kv_decode_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache, const float* k_scale,
                                const int8_t* v_cache, const float* v_scale, int64_t num_blocks, int block_size,
                                const int32_t* block_table, int64_t block_table_stride, const int32_t* context_lens,
                                int max_context_len, float scale, void* out, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  DecodeArgs a{};
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_cache; a.v_scale = v_scale;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.out = (_Float16*)out;
  return decode_common(a, false, false, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, scale, workspace, workspace_bytes, stream);
}

static int decode_append_int8_impl(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                       int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_new_stride_b,
                                       int64_t k_new_stride_h, const void* v_new, int64_t v_new_stride_b,
                                       int64_t v_new_stride_h, int8_t* k_cache, float* k_scale, int8_t* v_cache,
                                       float* v_scale, int64_t num_blocks, int block_size, const int32_t* block_table,
                                       int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                                       float scale, void* out, void* workspace, int64_t workspace_bytes,
                                       void* stream, const int32_t* plan) {
  DecodeArgs a{};
  a.plan = plan;
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_cache; a.v_scale = v_scale;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.out = (_Float16*)out;
  a.k_new = (const _Float16*)k_new;
  a.v_new = (const _Float16*)v_new;
  a.kn_stride_b = k_new_stride_b;
  a.kn_stride_h = k_new_stride_h;
  a.vn_stride_b = v_new_stride_b;
  a.vn_stride_h = v_new_stride_h;
  return decode_common(a, false, true, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, scale, workspace, workspace_bytes, stream);
}

extern "C" int s8kv_decode_append_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                       int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_new_stride_b,
                                       int64_t k_new_stride_h, const void* v_new, int64_t v_new_stride_b,
                                       int64_t v_new_stride_h, int8_t* k_cache, float* k_scale, int8_t* v_cache,
                                       float* v_scale, int64_t num_blocks, int block_size, const int32_t* block_table,
                                       int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                                       float scale, void* out, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  return decode_append_int8_impl(q, batch, num_q_heads, num_kv_heads, head_dim, q_stride_b, q_stride_h, k_new,
                                 k_new_stride_b, k_new_stride_h, v_new, v_new_stride_b, v_new_stride_h, k_cache,
                                 k_scale, v_cache, v_scale, num_blocks, block_size, block_table, block_table_stride,
                                 context_lens, max_context_len, scale, out, workspace, workspace_bytes, stream,
                                 nullptr);
}

extern "C" int s8kv_decode_append_int8_planned(const void* q, int batch, int num_q_heads, int num_kv_heads,
                                               int head_dim, int64_t q_stride_b, int64_t q_stride_h,
                                               const void* k_new, int64_t k_new_stride_b, int64_t k_new_stride_h,
                                               const void* v_new, int64_t v_new_stride_b, int64_t v_new_stride_h,
                                               int8_t* k_cache, float* k_scale, int8_t* v_cache, float* v_scale,
                                               int64_t num_blocks, int block_size, const int32_t* block_table,
                                               int64_t block_table_stride, const int32_t* context_lens,
                                               int max_context_len, float scale, void* out, void* workspace,
                                               int64_t workspace_bytes, void* stream, const void* plan,
                                               int64_t plan_bytes) {
  S8KV_REQUIRE(plan != nullptr && (uintptr_t)plan % 4 == 0, S8KV_ERR_INVALID,
               "decode_append_int8_planned: null or unaligned plan");
  S8KV_REQUIRE(plan_bytes >= plan_bytes_for(num_kv_heads), S8KV_ERR_INVALID,
               "decode_append_int8_planned: a plan of %lld bytes is needed, %lld given",
               (long long)plan_bytes_for(num_kv_heads), (long long)plan_bytes);
  return decode_append_int8_impl(q, batch, num_q_heads, num_kv_heads, head_dim, q_stride_b, q_stride_h, k_new,
                                 k_new_stride_b, k_new_stride_h, v_new, v_new_stride_b, v_new_stride_h, k_cache,
                                 k_scale, v_cache, v_scale, num_blocks, block_size, block_table, block_table_stride,
                                 context_lens, max_context_len, scale, out, workspace, workspace_bytes, stream,
                                 static_cast<const int32_t*>(plan));
}

extern "C" int s8kv_decode_append_int8_noalloc(const void* q, int batch, int num_q_heads, int num_kv_heads,
                                               int head_dim, int64_t q_stride_b, int64_t q_stride_h,
                                               const void* k_new, int64_t k_new_stride_b, int64_t k_new_stride_h,
                                               const void* v_new, int64_t v_new_stride_b, int64_t v_new_stride_h,
                                               int8_t* k_cache, float* k_scale, int8_t* v_cache, float* v_scale,
                                               int64_t num_blocks, int block_size, const int32_t* block_table,
                                               int64_t block_table_stride, const int32_t* context_lens,
                                               int max_context_len, float scale, void* out, void* stream) {
  if (batch > 0 && num_kv_heads > 0 && num_q_heads > 0 && head_dim > 0) {
    const int64_t need = workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim);
    S8KV_REQUIRE(need <= kScratchBytes, S8KV_ERR_WORKSPACE,
                 "decode_append_int8_noalloc: this geometry (batch %d, %d q heads, %d kv heads, head_dim %d) needs "
                 "%lld bytes of scratch, more than the %lld-byte static scratch; use s8kv_decode_append_int8",
                 batch, num_q_heads, num_kv_heads, head_dim, (long long)need, (long long)kScratchBytes);
  }
  void* ws = nullptr;
  if (batch > 0) {
    const int rc = scratch_for_current_device(&ws);
    if (rc != S8KV_OK) return rc;
  }
  DecodeArgs a{};
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_cache; a.v_scale = v_scale;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.out = (_Float16*)out;
  a.k_new = (const _Float16*)k_new;
  a.v_new = (const _Float16*)v_new;
  a.kn_stride_b = k_new_stride_b;
  a.kn_stride_h = k_new_stride_h;
  a.vn_stride_b = v_new_stride_b;
  a.vn_stride_h = v_new_stride_h;
  a.untimed = 1;
  return decode_common(a, false, true, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, scale, ws, kScratchBytes, stream);
}

static int decode_append_k8v3_impl(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                       int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_new_stride_b,
                                       int64_t k_new_stride_h, const void* v_new, int64_t v_new_stride_b,
                                       int64_t v_new_stride_h, int8_t* k_cache, float* k_scale, int32_t* v_packed,
                                       float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                                       int block_size, const int32_t* block_table, int64_t block_table_stride,
                                       const int32_t* context_lens, int max_context_len, float scale, void* out,
                                       void* workspace, int64_t workspace_bytes, void* stream, const int32_t* plan) {
  S8KV_REQUIRE(lloyd_block == 128, S8KV_ERR_UNSUPPORTED, "decode_append_k8v3: lloyd_block %d != 128", lloyd_block);
  S8KV_REQUIRE(v_codebook != nullptr, S8KV_ERR_INVALID, "decode_append_k8v3: null codebook");
  DecodeArgs a{};
  a.plan = plan;
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_packed; a.v_scale = v_norm;
  a.v_codebook = v_codebook;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.out = (_Float16*)out;
  a.k_new = (const _Float16*)k_new;
  a.v_new = (const _Float16*)v_new;
  a.kn_stride_b = k_new_stride_b;
  a.kn_stride_h = k_new_stride_h;
  a.vn_stride_b = v_new_stride_b;
  a.vn_stride_h = v_new_stride_h;
  return decode_common(a, true, true, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, scale, workspace, workspace_bytes, stream);
}

extern "C" int s8kv_decode_append_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                       int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_new_stride_b,
                                       int64_t k_new_stride_h, const void* v_new, int64_t v_new_stride_b,
                                       int64_t v_new_stride_h, int8_t* k_cache, float* k_scale, int32_t* v_packed,
                                       float* v_norm, const float* v_codebook, int lloyd_block, int64_t num_blocks,
                                       int block_size, const int32_t* block_table, int64_t block_table_stride,
                                       const int32_t* context_lens, int max_context_len, float scale, void* out,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  return decode_append_k8v3_impl(q, batch, num_q_heads, num_kv_heads, head_dim, q_stride_b, q_stride_h, k_new,
                                 k_new_stride_b, k_new_stride_h, v_new, v_new_stride_b, v_new_stride_h, k_cache,
                                 k_scale, v_packed, v_norm, v_codebook, lloyd_block, num_blocks, block_size,
                                 block_table, block_table_stride, context_lens, max_context_len, scale, out,
                                 workspace, workspace_bytes, stream, nullptr);
}

extern "C" int s8kv_decode_append_k8v3_planned(const void* q, int batch, int num_q_heads, int num_kv_heads,
                                               int head_dim, int64_t q_stride_b, int64_t q_stride_h,
                                               const void* k_new, int64_t k_new_stride_b, int64_t k_new_stride_h,
                                               const void* v_new, int64_t v_new_stride_b, int64_t v_new_stride_h,
                                               int8_t* k_cache, float* k_scale, int32_t* v_packed, float* v_norm,
                                               const float* v_codebook, int lloyd_block, int64_t num_blocks,
                                               int block_size, const int32_t* block_table, int64_t block_table_stride,
                                               const int32_t* context_lens, int max_context_len, float scale,
                                               void* out, void* workspace, int64_t workspace_bytes, void* stream,
                                               const void* plan,
                                               int64_t plan_bytes) {
  S8KV_REQUIRE(plan != nullptr && (uintptr_t)plan % 4 == 0, S8KV_ERR_INVALID,
               "decode_append_k8v3_planned: null or unaligned plan");
  S8KV_REQUIRE(plan_bytes >= plan_bytes_for(num_kv_heads), S8KV_ERR_INVALID,
               "decode_append_k8v3_planned: a plan of %lld bytes is needed, %lld given",
               (long long)plan_bytes_for(num_kv_heads), (long long)plan_bytes);
  return decode_append_k8v3_impl(q, batch, num_q_heads, num_kv_heads, head_dim, q_stride_b, q_stride_h, k_new,
                                 k_new_stride_b, k_new_stride_h, v_new, v_new_stride_b, v_new_stride_h, k_cache,
                                 k_scale, v_packed, v_norm, v_codebook, lloyd_block, num_blocks, block_size,
                                 block_table, block_table_stride, context_lens, max_context_len, scale, out,
                                 workspace, workspace_bytes, stream, static_cast<const int32_t*>(plan));
}

extern "C" int64_t s8kv_decode_plan_size(int num_kv_heads) {
  return num_kv_heads > 0 ? plan_bytes_for(num_kv_heads) : 0;
}

static int decode_plan_common(int batch, int num_q_heads, int num_kv_heads, int head_dim, int layout, int fused,
                              int64_t num_blocks, int block_size, const int32_t* block_table,
                              int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                              void* plan, int64_t plan_bytes_given, void* stream, bool adaptive) {
  S8KV_REQUIRE(layout == 0 || layout == 1, S8KV_ERR_INVALID, "decode_plan: layout %d is neither 0 (int8) nor 1 (k8v3)",
               layout);
  S8KV_REQUIRE(plan != nullptr, S8KV_ERR_INVALID, "decode_plan: null plan");
  DecodeArgs a{};
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.plan_out = static_cast<int32_t*>(plan);
  a.plan_adapt = adaptive ? 1 : 0;
  a.untimed = 1;
  return decode_common(a, layout == 1, fused != 0, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, 1.0f, plan, plan_bytes_given, stream);
}
extern "C" int s8kv_decode_plan(int batch, int num_q_heads, int num_kv_heads, int head_dim, int layout, int fused,
                                int64_t num_blocks, int block_size, const int32_t* block_table,
                                int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                                void* plan, int64_t plan_bytes_given, void* stream) {
  return decode_plan_common(batch, num_q_heads, num_kv_heads, head_dim, layout, fused, num_blocks, block_size,
                            block_table, block_table_stride, context_lens, max_context_len, plan, plan_bytes_given,
                            stream, false);
}
extern "C" int s8kv_decode_plan_adaptive(int batch, int num_q_heads, int num_kv_heads, int head_dim, int layout,
                                         int fused, int64_t num_blocks, int block_size, const int32_t* block_table,
                                         int64_t block_table_stride, const int32_t* context_lens,
                                         int max_context_len, void* plan, int64_t plan_bytes_given, void* stream) {
  return decode_plan_common(batch, num_q_heads, num_kv_heads, head_dim, layout, fused, num_blocks, block_size,
                            block_table, block_table_stride, context_lens, max_context_len, plan, plan_bytes_given,
                            stream, true);
}

extern "C" int s8kv_decode_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache, const float* k_scale,
                                const int32_t* v_packed, const float* v_norm, const float* v_codebook, int lloyd_block,
                                int64_t num_blocks, int block_size, const int32_t* block_table,
                                int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                                float scale, void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  S8KV_REQUIRE(lloyd_block == 128, S8KV_ERR_UNSUPPORTED, "decode_k8v3: lloyd_block %d != 128", lloyd_block);
  S8KV_REQUIRE(v_codebook != nullptr, S8KV_ERR_INVALID, "decode_k8v3: null codebook");
  DecodeArgs a{};
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_packed; a.v_scale = v_norm;
  a.v_codebook = v_codebook;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.out = (_Float16*)out;
  return decode_common(a, true, false, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, scale, workspace, workspace_bytes, stream);
}

extern "C" int s8kv_decode_window_int8(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                       int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache,
                                       const float* k_scale, const int8_t* v_cache, const float* v_scale,
                                       int64_t num_blocks, int block_size, const int32_t* block_table,
                                       int64_t block_table_stride, const int32_t* context_lens, int max_context_len,
                                       int window, float scale, void* out, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  S8KV_REQUIRE(window >= 1, S8KV_ERR_INVALID, "decode_window: window %d < 1", window);
  DecodeArgs a{};
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_cache; a.v_scale = v_scale;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.out = (_Float16*)out;
  a.window = window;
  return decode_common(a, false, false, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, scale, workspace, workspace_bytes, stream);
}

extern "C" int s8kv_decode_window_k8v3(const void* q, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                       int64_t q_stride_b, int64_t q_stride_h, const int8_t* k_cache,
                                       const float* k_scale, const int32_t* v_packed, const float* v_norm,
                                       const float* v_codebook, int lloyd_block, int64_t num_blocks, int block_size,
                                       const int32_t* block_table, int64_t block_table_stride,
                                       const int32_t* context_lens, int max_context_len, int window, float scale,
                                       void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  S8KV_REQUIRE(window >= 1, S8KV_ERR_INVALID, "decode_window: window %d < 1", window);
  S8KV_REQUIRE(lloyd_block == 128, S8KV_ERR_UNSUPPORTED, "decode_k8v3: lloyd_block %d != 128", lloyd_block);
  S8KV_REQUIRE(v_codebook != nullptr, S8KV_ERR_INVALID, "decode_k8v3: null codebook");
  DecodeArgs a{};
  a.q = (const _Float16*)q;
  a.q_stride_b = q_stride_b;
  a.q_stride_h = q_stride_h;
  a.k_cache = k_cache; a.k_scale = k_scale; a.v_cache = v_packed; a.v_scale = v_norm;
  a.v_codebook = v_codebook;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.out = (_Float16*)out;
  a.window = window;
  return decode_common(a, true, false, batch, num_q_heads, num_kv_heads, head_dim, num_blocks, block_size,
                       max_context_len, scale, workspace, workspace_bytes, stream);
}
