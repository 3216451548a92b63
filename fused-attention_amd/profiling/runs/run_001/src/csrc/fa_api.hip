// fa_api.hip - the extern "C" entry points declared in include/fa.h.
//
// Argument checking mirrors the reference's host wrappers
// (attention/fused/fused.py:69-71, attention/gqa/fused_gqa.py:71-77,
// attention/backward/fused_backward.py:151-158); the Python layer raises the
// reference's exception types before it ever reaches this ABI, so these
// checks are the last line of defence for C callers.
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
  if (!tile_ok(block_m) || !tile_ok(block_n)) return FA_ERR_TILE;
  if (S % block_m != 0 || S % block_n != 0) return FA_ERR_TILE;
  // element offsets inside one tensor are formed in 32-bit for the per-row
  // parts and 64-bit for the (batch, head) base; keep the whole tensor
  // addressable with 32-bit row indices
  if ((long long)B * H * S > 0x7fffffffLL) return FA_ERR_DIMS;
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
  const int gh = heads_per_wg(H / H_kv, block_m, block_n);
  fa::FwdFn fn = fwd_table(dtype, D, block_m, block_n, gh, lse != nullptr);
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
  fa::BwdFn fn = bwd_table(dtype, D, block_m, block_n);
  if (!fn) return FA_ERR_UNSUPPORTED;
  fa::BwdArgs a{q, k, v, o, d_o, lse, dq, dk, dv, B, H, H, S, D, scale_log2, sm_scale, hip_stream};
  return fn(a);
}

int fa_bwd_gqa(const void* q, const void* k, const void* v, const void* o,
               const void* d_o, const float* lse, void* dq, void* dk, void* dv,
               int B, int H, int H_kv, int S, int D, int dtype, float scale_log2, float sm_scale,
               int block_m, int block_n, void* hip_stream) {
  int st = check_common(B, H, S, D, dtype, block_m, block_n);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H_kv > H || H % H_kv != 0) return FA_ERR_DIMS;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv) return FA_ERR_NULL;
  fa::BwdFn fn = bwd_table(dtype, D, block_m, block_n);
  if (!fn) return FA_ERR_UNSUPPORTED;
  fa::BwdArgs a{q, k, v, o, d_o, lse, dq, dk, dv, B, H, H_kv, S, D, scale_log2, sm_scale, hip_stream};
  return fn(a);
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
    case FA_ERR_DIMS: return "invalid dimensions (B, H, H_kv, S must be positive and H_kv must divide H)";
    case FA_ERR_DTYPE: return "unsupported dtype (expected float16 or bfloat16)";
    case FA_ERR_HEADDIM: return "unsupported head dim (expected 32, 64 or 128)";
    case FA_ERR_TILE: return "unsupported tile (block_m and block_n must be 64 or 128 and divide S)";
    case FA_ERR_NULL: return "a required pointer is NULL";
    case FA_ERR_LAUNCH: return "HIP kernel launch failed";
    case FA_ERR_UNSUPPORTED: return "no kernel for this combination";
    default: return "unknown status";
  }
}

int fa_version(void) { return 110; }

}  // extern "C"
