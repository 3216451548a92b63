// fa_api.hip - the extern "C" entry points declared in include/fa.h.
//
// Argument checking mirrors the reference's host wrappers
// (attention/fused/fused.py:69-71, attention/gqa/fused_gqa.py:71-77,
// attention/backward/fused_backward.py:151-158); the Python layer raises the
// reference's exception types before it ever reaches this ABI, so these
// checks are the last line of defence for C callers.
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>

#include "fa_launch.h"

namespace {

constexpr int kMaxGroupHeadsPerWg = 4;

bool tile_ok(int t) { return t == 64 || t == 128; }

fa::FwdFn fwd_table(int dtype, int D, int bm, int bn, int gh, int lse) {
  if (dtype == FA_F16) {
    if (D == 32) return fa_fwd_table_f16_32(bm, bn, gh, lse);
    if (D == 64) return fa_fwd_table_f16_64(bm, bn, gh, lse);
    if (D == 128) return fa_fwd_table_f16_128(bm, bn, gh, lse);
  } else if (dtype == FA_BF16) {
    if (D == 32) return fa_fwd_table_bf16_32(bm, bn, gh, lse);
    if (D == 64) return fa_fwd_table_bf16_64(bm, bn, gh, lse);
    if (D == 128) return fa_fwd_table_bf16_128(bm, bn, gh, lse);
  }
  return nullptr;
}

fa::BwdFn bwd_table(int dtype, int D, int bm, int bn) {
  if (dtype == FA_F16) {
    if (D == 32) return fa_bwd_table_f16_32(bm, bn);
    if (D == 64) return fa_bwd_table_f16_64(bm, bn);
    if (D == 128) return fa_bwd_table_f16_128(bm, bn);
  } else if (dtype == FA_BF16) {
    if (D == 32) return fa_bwd_table_bf16_32(bm, bn);
    if (D == 64) return fa_bwd_table_bf16_64(bm, bn);
    if (D == 128) return fa_bwd_table_bf16_128(bm, bn);
  }
  return nullptr;
}

// Query heads per workgroup for a GQA group: as many heads of one K/V group
// as fit in 8 waves (512 threads), each head taking block_m/32 waves.  With
// 128-key tiles a wave holds two 128-key score tiles in flight and needs more
// than the 256 VGPRs of two waves per SIMD, so the workgroup stays at 4 waves.
// Counters (profiles/tile_study_mha_gqa_bwd.md, GQA B=2 H=32 H_kv=8 S=8192 D=128):
// one head of 64 rows 898 TFLOP/s, MFMA busy 48.2 %; two heads 1185 / 71.4 %; four
// heads 1236 / 68.4 %.
int heads_per_wg(int group, int block_m, int block_n) {
  int cap = (block_n == 128 ? 128 : 256) / block_m;  // waves / (block_m / 32)
  if (cap > kMaxGroupHeadsPerWg) cap = kMaxGroupHeadsPerWg;
  int gh = 1;
  while (gh * 2 <= cap && group % (gh * 2) == 0) gh *= 2;
  return gh;
}

int check_common(int B, int H, int S, int D, int dtype, int block_m, int block_n) {
  if (B <= 0 || H <= 0 || S <= 0) return FA_ERR_DIMS;
  if (dtype != FA_F16 && dtype != FA_BF16) return FA_ERR_DTYPE;
  if (D != 32 && D != 64 && D != 128) return FA_ERR_HEADDIM;
  if (!tile_ok(block_m) || !tile_ok(block_n)) return FA_ERR_TILE;  // any S >= 1: partial edge tiles
  // element offsets inside one tensor are formed in 32-bit for the per-row
  // parts and 64-bit for the (batch, head) base; keep the whole tensor
  // addressable with 32-bit row indices
  if ((long long)B * H * S > 0x7fffffffLL) return FA_ERR_DIMS;
  // the kernels form byte offsets inside one (batch, head) slice, and the byte
  // size of a slice's remaining rows, in 32-bit int: keep S * D * 2 below 2^31
  if ((long long)S * D * 2 > 0x7fffffffLL) return FA_ERR_DIMS;
  return FA_OK;
}

using fa::cu_count;
using fa::kMaxDevices;

// Forward query heads per workgroup for this launch: heads_per_wg's choice, but four
// heads (64-row tiles) drop to two where the grid would leave the co-resident pair of
// workgroups per CU short: below two workgroups per CU, and at D = 32 below four, where
// the heavy-first order cannot balance the causal triangle with the fewer, longer
// workgroups.  Two heads of 64 rows still hold two waves per SIMD.  Measured
// (profiles/tile_study_mha_gqa_bwd.md, TFLOP/s of two / four heads): B=1 H=16 H_kv=4
// S=4096 D=128 (one workgroup per CU at four heads) 864 / 754; B=2 H=8 H_kv=1 S=8192 fp16
// (two per CU) D=128 1045 / 1134, D=64 899 / 915, D=32 650 / 602; the study's run before
// it read the same order (D=128 990 / 1053, D=64 868 / 897, D=32 662 / 629).
// A 128-row tile with 64 keys runs as 64-row workgroups of four heads wherever the
// 64-row tile would take four: each K/V tile is then staged for four heads instead of
// two, and every 32-row wave computes the same either way (results bitwise equal).
// Interleaved timings, two heads of 128 rows against four of 64: GQA B=2 H=32 H_kv=8
// S=8192 D=128 +0.8 %, B=1 H=32 H_kv=4 S=8192 +0.9 %, B=2 H=32 H_kv=8 S=4096 +1.5 %,
// MQA B=1 H=32 S=16384 D=64 fp16 +0.3 %, B=2 H=32 H_kv=8 S=8192 D=64 fp16 +0.7 %.
int fwd_heads_per_wg(int B, int H, int group, int S, int D, int block_m, int block_n) {
  auto four_fit = [&](int bm) {
    return (long long)B * (H / 4) * ((S + bm - 1) / bm) >= (D <= 32 ? 4LL : 2LL) * cu_count();
  };
  if (block_m == 128 && block_n == 64 && heads_per_wg(group, 64, 64) == 4 && four_fit(64)) return 4;
  int gh = heads_per_wg(group, block_m, block_n);
  if (gh == 4 && !four_fit(block_m)) gh = 2;
  return gh;
}

// tile_m only sets how many 32-row waves share a workgroup: each 32-row group runs
// the same arithmetic over the same key tiles either way, so results do not depend
// on it (bitwise).  A single-head workgroup of 64 rows holds two waves, and with
// its K and V tiles double-buffered in LDS it gets one wave per SIMD or less;
// where that is measured slower, tile_m = 64 runs as 128-row workgroups.
// Forward, MHA B=4 H=32 S=4096 bf16, TFLOP/s of tile 64 -> 128 rows
// (profiles/tile_study_mha_gqa_bwd.md): tile_n = 64: D=128 845 -> 1106 (MFMA busy
// 43.9 -> 66.8 %: a 64-row workgroup holds one wave per SIMD), D=64 649 -> 922, D=32
// 441 -> 675; tile_n = 128: D=128 464 -> 775, D=64 631 -> 654, D=32 447 -> 461 (the
// D <= 64 forward at 128 keys +1.7-3.6 % at six shapes of A/B runs, -0.3 % at
// B=4 H=32 D=32 bf16; four runs of the study read 128 rows 2-5 % faster).  dQ, every
// head dim: 64 -> 128 rows at D=128 870 -> 1144 (MFMA busy 42.4 -> 62.2 %), at D=64
// 973 -> 1003 with 64-key tiles and 681 -> 1019 with 128-key tiles, at D=32 739 -> 794
// (the D = 32 backward +0.9-2.3 % at four shapes in A/B runs, -0.3 % at B=2 H=16 S=4096).
int fwd_block_m(int block_m, int /*block_n*/, int /*D*/, int gh) {
  if (gh == 4) return 64;  // four heads run 64-row tiles (fwd_heads_per_wg)
  return (block_m == 64 && gh == 1) ? 128 : block_m;
}
int dq_block_m(int block_m, int /*D*/) { return block_m == 64 ? 128 : block_m; }

// Work items (key-tile chunks) the dK/dV kernel should have for its heavy-first order
// to balance: two per workgroup slot the GPU holds at once, and one round more per
// 8192 keys beyond, since the heaviest key tile's pairs grow with S while the average
// does not keep up (a split costs an fp32 partial write, read and reduction, so it is
// kept to what load balance needs).  Slots: the paired D = 128 kernel runs one
// persistent workgroup per CU that walks its items; the one-wave kernel (D <= 64) two
// workgroups per CU, one per item.  Measured (profiles/dkdv_split_study.md, dK/dV +
// reduction, us, the rule's choice first):
//   paired: MQA B=1 H=32 S=4096 D=128, 16 / 8 / 32: 253 / 377 / 280; MHA B=1 H=4 S=8192,
//   2 / 1 / 4: 140 / 197 / 160; MHA B=1 H=8 S=4096, 2 / 1 / 4: 84 / 95 / 105; GQA B=1 H=32
//   H_kv=4 S=8192, 2 / 1 / 4: 913 / 1427 / 937; B=1 H=8 H_kv=1 S=16384, 8 / 4 / 16: 920 /
//   1170 / 965;
//   one-wave: MQA B=1 H=32 S=4096 D=64, 32 / 16 / 64: 179 / 212 / 188; MHA B=1 H=16 S=4096
//   D=64, 2 / 1 / 4: 98 / 108 / 113; B=2 H=16 S=4096 D=64, 1 / 2: 155 / 186; MQA B=1 H=32
//   S=16384 D=64, 16 / 8 / 32: 2039 / 2160 / 2074.
// (The previous rule, 2 x CU items per 4096 keys for both kernels, chose 4 for MHA
// B=1 H=4 S=8192 and for the GQA shape, 16 for B=1 H=8 H_kv=1 and for MQA S=4096 D=64, and
// 1 for MHA B=1 H=16 D=64: 14, 3, 5, 18 and 10 % slower.)  D = 32 runs the one-wave kernel
// and takes its rule unmeasured.
int dkdv_target_workgroups(int S, int D) {
  const int slots = cu_count() * (D == 128 ? 1 : 2);
  return 2 * slots * std::max(1, (S + 8191) / 8192);
}

size_t gqa_workspace_bytes(int B, int H_kv, int S, int D, int nsplit) {
  return nsplit > 1 ? 2 * (size_t)B * H_kv * nsplit * S * D * sizeof(float) : 0;
}

// -LSE/c and -Delta per query row ([2, B*H, S] fp32), rounded up to 256 bytes so
// the partial sums after them stay aligned
size_t rowb_bytes(int B, int H, int S) {
  return (2 * (size_t)B * H * S * sizeof(float) + 255) / 256 * 256;
}

// Chunks per key tile for dK/dV: enough that B * H_kv * (key tiles) * nsplit
// reaches the target number of work items, at most the pairs of the heaviest key
// tile (G query heads x all 64-row query tiles) and kMaxDkdvSplit; 1 when the key
// tiles alone already reach it, or when the heaviest tile has fewer than
// kMinSplitPairs pairs: then the partial-sum traffic and the extra pass cost more
// than the imbalance (profiles/tile_study_mha_gqa_bwd.md, dK/dV + reduction: B=2 H=8
// S=2048 D=128, 32 pairs, 57 us whole against 282 at split 16; B=1 H=8 S=4096, 64
// pairs, 98 -> 86 us at split 2; MQA B=1 H=32 S=4096 D=64 1748 -> 196 us at split 64).
constexpr int kMaxDkdvSplit = 64;
constexpr int kMinSplitPairs = 64;
int dkdv_nsplit(int B, int H, int H_kv, int S, int D) {
  const long long items = (long long)B * H_kv * ((S + fa::kDkdvKeys - 1) / fa::kDkdvKeys);
  const long long want = dkdv_target_workgroups(S, D);
  const long long pairs = (long long)(H / H_kv) * ((S + 63) / 64);
  if (items >= want || pairs < kMinSplitPairs) return 1;
  long long s = (want + items - 1) / items;
  if (s > pairs) s = pairs;
  if (s > kMaxDkdvSplit) s = kMaxDkdvSplit;
  return s < 1 ? 1 : (int)s;
}

// ---------------------------------------------------------------------------
// Device scratch of the allocation-free backward (fa_bwd_gqa_noalloc): stands in
// for fa_bwd_gqa's caller workspace.  Each device that loads the library holds its
// own copy until the process ends.  On the host the array's name is only a
// stand-in for the symbol, never a device address: host code uses the address
// that hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

// This device's copy of `scratch`, looked up on the first call on the device (with
// it current) and kept; FA_ERR_LAUNCH if the runtime cannot name it.
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FA_ERR_LAUNCH;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return FA_ERR_LAUNCH;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FA_OK;
}

}  // namespace

extern "C" {

int fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
           int B, int H, int H_kv, int S, int D, int dtype, float scale_log2,
           int block_m, int block_n, void* hip_stream) {
  int st = check_common(B, H, S, D, dtype, block_m, block_n);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H_kv > H || H % H_kv != 0) return FA_ERR_DIMS;
  if (!q || !k || !v || !o) return FA_ERR_NULL;
  const int gh = fwd_heads_per_wg(B, H, H / H_kv, S, D, block_m, block_n);
  fa::FwdFn fn = fwd_table(dtype, D, fwd_block_m(block_m, block_n, D, gh), block_n, gh, lse != nullptr);
  if (!fn) return FA_ERR_UNSUPPORTED;
  fa::FwdArgs a{q, k, v, o, lse, B, H, H_kv, S, D, scale_log2, hip_stream};
  return fn(a);
}

int fa_bwd(const void* q, const void* k, const void* v, const void* o,
           const void* d_o, const float* lse, void* dq, void* dk, void* dv,
           int B, int H, int S, int D, int dtype, float scale_log2, float sm_scale,
           int block_m, int block_n, void* hip_stream) {
  int st = check_common(B, H, S, D, dtype, block_m, block_n);
  if (st != FA_OK) return st;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv) return FA_ERR_NULL;
  fa::BwdFn fn = bwd_table(dtype, D, dq_block_m(block_m, D), block_n);
  if (!fn) return FA_ERR_UNSUPPORTED;
  fa::BwdArgs a{q, k, v, o, d_o, lse, dq, dk, dv, B, H, H, S, D, scale_log2, sm_scale, hip_stream,
                nullptr, nullptr, 1, nullptr, false};
  return fn(a);
}

size_t fa_bwd_gqa_workspace_size(int B, int H, int H_kv, int S, int D) {
  if (B <= 0 || H <= 0 || S <= 0 || H_kv <= 0 || H_kv > H || H % H_kv != 0) return 0;
  if (D != 32 && D != 64 && D != 128) return 0;
  return rowb_bytes(B, H, S) + gqa_workspace_bytes(B, H_kv, S, D, dkdv_nsplit(B, H, H_kv, S, D));
}

int fa_bwd_gqa(const void* q, const void* k, const void* v, const void* o,
               const void* d_o, const float* lse, void* dq, void* dk, void* dv,
               int B, int H, int H_kv, int S, int D, int dtype, float scale_log2, float sm_scale,
               int block_m, int block_n, void* workspace, size_t workspace_bytes, void* hip_stream) {
  int st = check_common(B, H, S, D, dtype, block_m, block_n);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H_kv > H || H % H_kv != 0) return FA_ERR_DIMS;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv) return FA_ERR_NULL;
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15)) return FA_ERR_WORKSPACE;
  fa::BwdFn fn = bwd_table(dtype, D, dq_block_m(block_m, D), block_n);
  if (!fn) return FA_ERR_UNSUPPORTED;
  // the workspace holds, in this order and as far as it reaches: the per-row terms
  // (dQ then runs first and dK/dV reads Delta instead of forming it), then the
  // partial sums of the split the shape asks for, or of the largest one that fits
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  size_t left = workspace ? workspace_bytes : 0;
  float* rowb = nullptr;
  if (left >= rowb_bytes(B, H, S)) {
    rowb = reinterpret_cast<float*>(ws);
    ws += rowb_bytes(B, H, S);
    left -= rowb_bytes(B, H, S);
  }
  int nsplit = workspace ? dkdv_nsplit(B, H, H_kv, S, D) : 1;
  while (nsplit > 1 && gqa_workspace_bytes(B, H_kv, S, D, nsplit) > left) --nsplit;
  float* wsk = nsplit > 1 ? reinterpret_cast<float*>(ws) : nullptr;
  float* wsv = nsplit > 1 ? wsk + (size_t)B * H_kv * nsplit * S * D : nullptr;
  fa::BwdArgs a{q, k, v, o, d_o, lse, dq, dk, dv, B, H, H_kv, S, D, scale_log2, sm_scale, hip_stream,
                wsk, wsv, nsplit, rowb, false};
  return fn(a);
}

int fa_bwd_gqa_noalloc(const void* q, const void* k, const void* v, const void* o,
                       const void* d_o, const float* lse, void* dq, void* dk, void* dv,
                       int B, int H, int H_kv, int S, int D, int dtype, float scale_log2, float sm_scale,
                       int block_m, int block_n, void* hip_stream) {
  int st = check_common(B, H, S, D, dtype, block_m, block_n);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H_kv > H || H % H_kv != 0) return FA_ERR_DIMS;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv) return FA_ERR_NULL;
  // the scratch is fa_bwd_gqa's workspace of kNoAllocScratchBytes: the per-row terms must
  // fit, and fa_bwd_gqa then takes the largest dK/dV split whose partial sums fit behind
  // them (the whole split the shape asks for when it fits), so the results are those of
  // fa_bwd_gqa given a workspace of that size.  Nothing in it needs clearing: dQ writes
  // every row's terms before dK/dV reads them, and every split chunk stores its whole
  // partial sum before the reduction reads it.
  if (rowb_bytes(B, H, S) > kNoAllocScratchBytes) return FA_ERR_SCRATCH;
  void* ws = nullptr;
  st = scratch_address(&ws);
  if (st != FA_OK) return st;
  return fa_bwd_gqa(q, k, v, o, d_o, lse, dq, dk, dv, B, H, H_kv, S, D, dtype, scale_log2, sm_scale,
                    block_m, block_n, ws, kNoAllocScratchBytes, hip_stream);
}

size_t fa_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int fa_fwd_exact(const void* q, const void* k, const void* v, void* o, float* lse,
                 int B, int H, int H_kv, int S, int D, int dtype, float scale_log2,
                 int block_m, int block_n, int heads_per_wg, void* hip_stream) {
  int st = check_common(B, H, S, D, dtype, block_m, block_n);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H_kv > H || H % H_kv != 0) return FA_ERR_DIMS;
  // the heads of one workgroup share one K/V head
  if (heads_per_wg <= 0 || (H / H_kv) % heads_per_wg != 0) return FA_ERR_DIMS;
  if (!q || !k || !v || !o) return FA_ERR_NULL;
  fa::FwdFn fn = fwd_table(dtype, D, block_m, block_n, heads_per_wg, lse != nullptr);
  if (!fn) return FA_ERR_UNSUPPORTED;
  fa::FwdArgs a{q, k, v, o, lse, B, H, H_kv, S, D, scale_log2, hip_stream};
  return fn(a);
}

int fa_bwd_gqa_exact(const void* q, const void* k, const void* v, const void* o,
                     const void* d_o, const float* lse, void* dq, void* dk, void* dv,
                     int B, int H, int H_kv, int S, int D, int dtype, float scale_log2, float sm_scale,
                     int dq_block_m, int dq_block_n, int nsplit, void* workspace, size_t workspace_bytes,
                     void* hip_stream) {
  int st = check_common(B, H, S, D, dtype, dq_block_m, dq_block_n);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H_kv > H || H % H_kv != 0) return FA_ERR_DIMS;
  if (nsplit < 1 || nsplit > kMaxDkdvSplit) return FA_ERR_DIMS;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv) return FA_ERR_NULL;
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15)) return FA_ERR_WORKSPACE;
  // the split's partial sums must fit behind the per-row terms; without a workspace
  // the reference's order runs (dK/dV forming Delta, then dQ)
  const size_t need = rowb_bytes(B, H, S) + gqa_workspace_bytes(B, H_kv, S, D, nsplit);
  if (nsplit > 1 && (!workspace || workspace_bytes < need)) return FA_ERR_WORKSPACE;
  fa::BwdFn fn = bwd_table(dtype, D, dq_block_m, dq_block_n);
  if (!fn) return FA_ERR_UNSUPPORTED;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const bool rows = workspace && workspace_bytes >= rowb_bytes(B, H, S);
  float* rowb = rows ? reinterpret_cast<float*>(ws) : nullptr;
  float* wsk = nsplit > 1 ? reinterpret_cast<float*>(ws + rowb_bytes(B, H, S)) : nullptr;
  float* wsv = nsplit > 1 ? wsk + (size_t)B * H_kv * nsplit * S * D : nullptr;
  fa::BwdArgs a{q, k, v, o, d_o, lse, dq, dk, dv, B, H, H_kv, S, D, scale_log2, sm_scale, hip_stream,
                wsk, wsv, nsplit, rowb, rowb == nullptr};
  return fn(a);
}

int fa_fwd_heads_per_wg(int B, int H, int H_kv, int S, int D, int block_m, int block_n) {
  if (B <= 0 || H <= 0 || S <= 0 || H_kv <= 0 || H_kv > H || H % H_kv != 0) return 0;
  if (D != 32 && D != 64 && D != 128) return 0;
  if (!tile_ok(block_m) || !tile_ok(block_n)) return 0;
  return fwd_heads_per_wg(B, H, H / H_kv, S, D, block_m, block_n);
}

int fa_fwd_rows_per_wg(int block_m, int block_n, int D, int heads_per_wg) {
  if (!tile_ok(block_m) || !tile_ok(block_n)) return 0;
  return fwd_block_m(block_m, block_n, D, heads_per_wg);
}

int fa_bwd_dq_rows_per_wg(int block_m, int D) { return tile_ok(block_m) ? dq_block_m(block_m, D) : 0; }

int fa_bwd_dkdv_split(int B, int H, int H_kv, int S, int D) {
  if (B <= 0 || H <= 0 || S <= 0 || H_kv <= 0 || H_kv > H || H % H_kv != 0) return 0;
  if (D != 32 && D != 64 && D != 128) return 0;
  return dkdv_nsplit(B, H, H_kv, S, D);
}

int fa_supported(int dtype, int D, int block_m, int block_n, int group, int with_lse, int is_bwd) {
  if (check_common(1, 1, 256, D, dtype, block_m, block_n) != FA_OK) return 0;
  if (group <= 0) return 0;
  if (is_bwd) return bwd_table(dtype, D, block_m, block_n) ? 1 : 0;
  return fwd_table(dtype, D, block_m, block_n, heads_per_wg(group, block_m, block_n), with_lse) ? 1 : 0;
}

const char* fa_strerror(int status) {
  switch (status) {
    case FA_OK: return "ok";
    case FA_ERR_DIMS:
      return "invalid dimensions (B, H, H_kv, S must be positive, H_kv must divide H, B*H*S and "
             "S*D*2 must stay below 2^31)";
    case FA_ERR_DTYPE: return "unsupported dtype (expected float16 or bfloat16)";
    case FA_ERR_HEADDIM: return "unsupported head dim (expected 32, 64 or 128)";
    case FA_ERR_TILE: return "unsupported tile (block_m and block_n must be 64 or 128)";
    case FA_ERR_NULL: return "a required pointer is NULL";
    case FA_ERR_LAUNCH: return "HIP kernel launch failed";
    case FA_ERR_UNSUPPORTED: return "no kernel for this combination";
    case FA_ERR_WORKSPACE:
      return "workspace not 16-byte aligned (or, for fa_bwd_gqa_exact, too small for the requested split)";
    case FA_ERR_SCRATCH:
      return "this shape's per-row terms (8 * B * H * S bytes) exceed the library's device scratch "
             "(fa_bwd_gqa_noalloc); use fa_bwd_gqa with a caller workspace";
    default: return "unknown status";
  }
}

int fa_version(void) { return 140; }

}  // extern "C"
