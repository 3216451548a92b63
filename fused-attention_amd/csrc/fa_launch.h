// fa_launch.h - host-side launch plumbing shared by the kernel translation units
// and the C ABI (fa_api.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include "../../include/fa.h"

namespace fa {

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int B, H, Hkv, S, D;
  float scale_log2;
  void* stream;
};

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* d_o;
  const float* lse;
  void* dq;
  void* dk;
  void* dv;
  int B, H, Hkv, S, D;
  float scale_log2;
  float sm_scale;
  void* stream;
  // the (query tile, query head) pairs of a key tile are split over `nsplit`
  // workgroups, each writing fp32 partial dK / dV ([B*Hkv*nsplit, S, D] each) that a
  // reduction pass adds up; nsplit = 1: one workgroup, no workspace
  float* wsk;
  float* wsv;
  int nsplit;
  // [2, B*H, S] fp32: -LSE/c and -Delta of every query row, written by the dQ
  // kernel (then launched first) for the dK/dV kernel; null: dK/dV runs first, with
  // the terms written into dQ's own buffer by a row-terms pass (dQ overwrites them
  // last), or, with form_delta, formed by the dK/dV kernel in every key tile
  float* rowb;
  bool form_delta;
};

// keys per dK/dV workgroup (4 waves x 32 keys), for the split heuristics on the host
constexpr int kDkdvKeys = 128;

typedef int (*FwdFn)(const FwdArgs&);
typedef int (*BwdFn)(const BwdArgs&);

// Raise the dynamic LDS limit of a kernel once (needed above 64 KB).  The
// static local makes the first call per kernel instance thread-safe.
template <int SMEM>
inline bool smem_attr(const void* kern) {
  if (SMEM <= 65536) return true;
  return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, SMEM) == hipSuccess;
}

// CU count of the current device, read once per device and kept (the launch paths ask
// on every call, and a short call is bound by host time).  A failed query is answered
// with 256 (an MI355X) and leaves the HIP error state as the query left it: nothing here
// clears an error the caller's own work left behind.
constexpr int kMaxDevices = 64;
inline int cu_count() {
  static std::atomic<int> cus_of[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int cus = cus_of[dev].load(std::memory_order_relaxed);
  if (cus > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  cus_of[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Grid of a kernel whose workgroups walk their share of `items` work items: the item
// count rounded up to a multiple of 8 (workgroups reach the 8 XCDs in turn), capped
// at the workgroups the device runs at once (its CUs times the kernel's occupancy
// per_cu, rounded down to a multiple of 8).
inline int resident_grid(int items, int per_cu) {
  const int all = (items + 7) / 8 * 8;
  if (per_cu <= 0) return all;
  const int resident = cu_count() * per_cu / 8 * 8;
  return resident >= 8 && resident < all ? resident : all;
}

// Workgroups of `kern` (launched with `threads` threads) that one CU holds at once;
// 0 if the runtime cannot tell (the callers keep the answer per kernel).
inline int occupancy_per_cu(const void* kern, int threads) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, 0) != hipSuccess) return 0;
  return per_cu;
}

#define set_smem_once(kern, SMEM)                                   \
  ([&]() {                                                          \
    static const bool ok_ = ::fa::smem_attr<SMEM>(kern);            \
    return ok_;                                                     \
  }())

}  // namespace fa

#define FA_HIDDEN __attribute__((visibility("hidden")))

// Per-slice dispatch tables, one translation unit per (element type, D).
extern "C" {
FA_HIDDEN fa::FwdFn fa_fwd_table_f16_32(int bm, int bn, int gh, int lse);
FA_HIDDEN fa::FwdFn fa_fwd_table_f16_64(int bm, int bn, int gh, int lse);
FA_HIDDEN fa::FwdFn fa_fwd_table_f16_128(int bm, int bn, int gh, int lse);
FA_HIDDEN fa::FwdFn fa_fwd_table_bf16_32(int bm, int bn, int gh, int lse);
FA_HIDDEN fa::FwdFn fa_fwd_table_bf16_64(int bm, int bn, int gh, int lse);
FA_HIDDEN fa::FwdFn fa_fwd_table_bf16_128(int bm, int bn, int gh, int lse);
FA_HIDDEN fa::BwdFn fa_bwd_table_f16_32(int bm, int bn);
FA_HIDDEN fa::BwdFn fa_bwd_table_f16_64(int bm, int bn);
FA_HIDDEN fa::BwdFn fa_bwd_table_f16_128(int bm, int bn);
FA_HIDDEN fa::BwdFn fa_bwd_table_bf16_32(int bm, int bn);
FA_HIDDEN fa::BwdFn fa_bwd_table_bf16_64(int bm, int bn);
FA_HIDDEN fa::BwdFn fa_bwd_table_bf16_128(int bm, int bn);
}
