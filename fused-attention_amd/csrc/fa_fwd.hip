// fa_fwd.hip - causal attention forward for gfx950 (MHA, GQA/MQA, optional LSE).
//
// Algorithm (the reference's online softmax, attention/fused/fused.py:11-65,
// attention/gqa/fused_gqa.py:12-67, attention/backward/fused_backward.py:26-62):
//   per query row: m = -inf, l = 0, acc = 0 (fp32)
//   for every key tile j up to the diagonal:
//     s = q . k                     (fp32 MFMA accumulation)
//     s = -inf where key > query    (only on tiles that straddle the diagonal)
//     m_new = max(m, rowmax(s) * c) with c = log2(e)/sqrt(D)
//     alpha = exp2(m - m_new); p = exp2(s*c - m_new)
//     P = p rounded to the input type
//     l = l*alpha + rowsum(P)
//     acc = acc*alpha + P . v
//   O = acc / l; optional LSE = m + log2(l) (fused_backward.py:169).
// Two differences from the reference's arithmetic, both far inside the fp32
// reference's tolerance: l sums the rounded P that the PV product uses (the
// reference sums the unrounded p, fused.py:59), so O is an exactly normalised
// average of the V rows it weights; and the running max is lazy: acc and l are
// rescaled only when some row's max grows by more than FA_RESCALE_THRESHOLD
// powers of two (p then stays <= 2^T).  O = acc / l and LSE = m + log2(l) do
// not depend on the reference point m, and because l sums the same rounded
// weights as acc, a row dominated by one key still reproduces that key's V row.
//
// MI355X mapping:
//   * one workgroup = GH query heads (sharing one K/V head) x BM query rows;
//     one wave = one head x 32 query rows; WR = BM/32 waves per head.
//   * each wave computes S^T = K Q^T (keys x queries) so a lane owns ONE query
//     row: row max / row sum are register-local plus one permlane32 swap, and the
//     score accumulator is fed straight back as the B operand of O^T += V^T P^T.
//   * Q stays in registers for the whole loop.  K and V tiles go global -> LDS
//     with buffer_load_dwordx4 ... lds (no VGPR staging; the per-lane source
//     offsets are fixed, the tile offset is a scalar), double-buffered in two
//     LDS arrays; the next tile's DMA runs while the current tile is computed.
//   * V^T operands come from ds_read_b64_tr_b16 on the row-major V tile, so no
//     transpose is ever materialised.
//   * causal skipping at two levels: key tiles past the workgroup's last row are
//     never loaded, and each wave skips 32-key blocks past its own last row;
//     tiles wholly below the diagonal run a mask-free path.
//   * heavy-first, XCD-aware order: the 8 XCDs each take a contiguous range of
//     (batch, head-group) units; inside a unit the last (heaviest) query tile
//     is dispatched first.
//
// LDS layouts (one buffer = K tile then V tile, each BN rows x D, row-major).
// gfx950's LDS has 64 banks of 4 bytes: a 16-byte read is served 16 lanes per
// cycle and an 8-byte read 16 lanes per cycle (measured: 16-byte reads stream at
// twice the bytes per clock of 8-byte reads), so a read is conflict free when
// the lanes of each 16-lane phase touch distinct banks.
//   K: 16-byte chunk ch of row r stored at chunk ch ^ kswz(r), kswz(r) =
//      (r * CPR / 16) & (CPR - 1) with CPR chunks per row; an MFMA A-operand
//      read (lane c reads row c, one chunk) then puts the 16 lanes of a phase
//      on 16 distinct 16-byte bank slots.
//   V: byte b of row r stored at b ^ (32 * (r & 3)); a transposed read (16 lanes
//      = 4 rows x 32 bytes) then hits 4 distinct 32-byte bank groups.
#include "fa_device.h"
#include "fa_launch.h"

namespace fa {

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima)
constexpr int kWaitVmcnt0 = 0x0F70;
// skip the rescale unless a row max grows by more than this (log2 units)
#ifndef FA_RESCALE_THRESHOLD
#define FA_RESCALE_THRESHOLD 8.0f
#endif
constexpr float kRescaleThreshold = FA_RESCALE_THRESHOLD;

template <int D, int BM, int BN, int GH>
constexpr int fwd_waves_per_simd() {
  return (BN == 64 && (BM / 32) * GH >= 4) ? 2 : 1;
}

template <bool B>
struct Tag {
  static constexpr bool value = B;
};

// Two 8-byte transposed LDS reads -> one 16-byte MFMA operand.
__device__ __forceinline__ u32x4 lds_read_tr16x2(const unsigned char* base, int off0, int off1) {
  i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + off0));
  i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + off1));
  u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return u32x4{ua[0], ua[1], ub[0], ub[1]};
}

template <typename E, int D, int BM, int BN, int GH, bool LSE>
__global__ __launch_bounds__(64 * (BM / 32) * GH)
__attribute__((amdgpu_waves_per_eu(fwd_waves_per_simd<D, BM, BN, GH>(), fwd_waves_per_simd<D, BM, BN, GH>())))
void fwd_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ Lse,
                int B, int H, int Hkv, int S, float scale_log2) {
  constexpr int WR = BM / 32;
  constexpr int NW = WR * GH;
  constexpr int NB = BN / 32;          // 32-key blocks per tile
  constexpr int KT = D / 16;           // MFMA k-steps over D
  constexpr int DB = D / 32;           // 32-row blocks of O^T
  constexpr int ROWB = D * 2;          // bytes per K/V row
  constexpr int TILE = BN * ROWB;      // bytes per K or V tile
  constexpr int NBLK = TILE / 1024;    // 1 KB DMA blocks per tile
  constexpr int CPR = ROWB / 16;       // 16-byte chunks per row
  constexpr int NDMA = (NBLK + NW - 1) / NW;  // DMA blocks per wave per tile (K and V each)
  static_assert(TILE % 1024 == 0, "tile must be whole 1 KB DMA blocks");
  const float NEG_INF = -__builtin_inff();

  __shared__ __attribute__((aligned(1024))) unsigned char lds0[2 * TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char lds1[2 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hh = lane >> 5;
  const int wh = wave % GH, wr = wave / GH;

  // ---- work item: (batch, head group, query tile), heavy first, XCD aware
  const int nq = S / BM;
  const int units_per_b = H / GH;
  const int total = B * units_per_b * nq;
  const int wg = blockIdx.x;
  const int L = (total % 8 == 0) ? (wg % 8) * (total / 8) + (wg / 8) : wg;
  const int unit = L / nq;
  const int qt = nq - 1 - (L % nq);
  const int b = unit / units_per_b;
  const int h0 = (unit % units_per_b) * GH;
  const int hq = h0 + wh;
  const int hkv = h0 / (H / Hkv);

  const unsigned char* Kbh = reinterpret_cast<const unsigned char*>(K + (size_t)(b * Hkv + hkv) * S * D);
  const unsigned char* Vbh = reinterpret_cast<const unsigned char*>(V + (size_t)(b * Hkv + hkv) * S * D);
  const size_t qbase = (size_t)(b * H + hq) * S * D;

  const int r0 = qt * BM;          // first query row of this workgroup
  const int q0 = r0 + wr * 32;     // first query row of this wave
  const int m = q0 + c;            // this lane's query row
  const int ntiles = (r0 + BM + BN - 1) / BN;
  const int jfull = r0 / BN;       // tiles wholly below the workgroup's first row

  // ---- DMA of one K/V tile into an LDS buffer: 1 KB per wave instruction,
  // lane L's 16 bytes land at block + 16 L; the lane loads the global bytes
  // that belong there under the swizzles above.  A lane's source offsets inside
  // a tile are fixed (kvo / vvo); the tile offset j*TILE is a scalar (soffset).
  const int drow = lane / CPR;                 // row inside a 1 KB block
  const int dpos = (lane % CPR) * 16;          // LDS byte offset inside the row
  int kvo[NDMA], vvo[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int row = (wave + i * NW) * (1024 / ROWB) + drow;
    kvo[i] = row * ROWB + (((dpos >> 4) ^ ((row * CPR / 16) & (CPR - 1))) << 4);
    vvo[i] = row * ROWB + (dpos ^ ((32 * (row & 3)) & (ROWB - 1)));
  }
  const auto krs = make_rsrc(Kbh, S * ROWB);
  const auto vrs = make_rsrc(Vbh, S * ROWB);
  auto dma_tile = [&](int j, unsigned char* buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int blk = wave + i * NW;
      if (NBLK % NW == 0 || blk < NBLK) {
        dma16(krs, buf + blk * 1024, kvo[i], j * TILE);
        dma16(vrs, buf + TILE + blk * 1024, vvo[i], j * TILE);
      }
    }
  };

  // ---- Q^T operand in registers: k-step t holds Q[m][16t + 8hh .. +7]
  u32x4 qf[KT];
  {
    const uint16_t* qrow = Q + qbase + (size_t)m * D + 8 * hh;
#pragma unroll
    for (int t = 0; t < KT; ++t) qf[t] = gload16(qrow + 16 * t);
  }
  dma_tile(0, lds0);

  // ---- per-lane LDS operand offsets
  // K A-operand, k-step t: row c (+ 32 nb), chunk (2t+hh) ^ kswz(c)
  int koff[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) koff[t] = c * ROWB + (((2 * t + hh) ^ ((c * CPR / 16) & (CPR - 1))) << 4);
  // V^T A-operand via transposed reads: in 16-lane group G, lane (kr, c4) addresses
  // key row 4hh + kr (+ block offsets) and the 4 columns feeding output lanes
  // 4c4..4c4+3, which hold d = pi(16(G&1) + 4c4) + 0..3 of the 32-d block.
  int voff_even, voff_odd;
  {
    const int G = lane >> 4, kr = (lane >> 2) & 3, c4 = lane & 3;
    const int e = 2 * pi_swap23(16 * (G & 1) + 4 * c4);     // byte offset < 64
    const int k1 = (ROWB >= 128) ? (kr >> 1) : 0;
    const int base = (4 * hh + kr) * ROWB + (e ^ (32 * (kr & 1)));
    voff_even = base + 64 * k1;           // (64 db + e) ^ 32 kr for even db, minus 64 db
    voff_odd = base + 64 * (1 - k1) - 64;  // same for odd db
  }

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
  float mrun = NEG_INF, lrun = 0.f;

  // ---- one key tile
  auto compute = [&](const unsigned char* Ks, int k0, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(mask_tag)::value;
    const unsigned char* Vs = Ks + TILE;
    int nvalid = NB;
    if constexpr (MASKED) {
      nvalid = (q0 + 32 - k0) / 32;
      nvalid = nvalid > NB ? NB : nvalid;
      if (nvalid <= 0) return;
    }

    // S^T = K Q^T: A row c <- key 32nb + c; register g of lane (c, hh) holds
    // key offset 8*(g/4) + 4*hh + (g%4) of the block, query c
    f32x16 s[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (!MASKED || nb < nvalid) {
        f32x16 x = f32x16{};
#pragma unroll
        for (int t = 0; t < KT; ++t)
          x = mfma32<E>(lds_read16(Ks, koff[t] + nb * 32 * ROWB), qf[t], x);
        s[nb] = x;
      }
    }

    float mx = NEG_INF;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (!MASKED || nb < nvalid) {
        if (MASKED && k0 + 32 * nb == q0) {
#pragma unroll
          for (int g = 0; g < 16; ++g) {
            const int koffs = 8 * (g >> 2) + 4 * hh + (g & 3);
            if (koffs > c) s[nb][g] = NEG_INF;
          }
        }
#pragma unroll
        for (int g = 0; g < 16; ++g) mx = fmaxf(mx, s[nb][g]);
      }
    }
    mx = halfwave_max(mx) * scale_log2;

    // move the reference max (and rescale) only when some row's max grows
    if (__builtin_amdgcn_ballot_w64(mx > mrun + kRescaleThreshold)) {
      const float mnew = fmaxf(mrun, mx);
      const float alpha = fast_exp2(mrun - mnew);
      mrun = mnew;
      lrun *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g = 0; g < 16; ++g) acc[db][g] *= alpha;
    }

    // P^T as the B operand of the PV MFMAs: k-step u = 2nb + i1 holds
    // keys 32nb + 16i1 + 4hh + {0..3} (slots 0-3) and +8 (slots 4-7)
    // l sums the rounded P two at a time (v_dot2c with (1, 1)).
    u32x4 pk[2 * NB];
    float lsum[2] = {0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (!MASKED || nb < nvalid) {
        float p[16];
#pragma unroll
        for (int g = 0; g < 16; ++g) p[g] = fast_exp2(__builtin_fmaf(s[nb][g], scale_log2, -mrun));
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) {
          u32x4 w;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            w[q] = pack2<E>(p[8 * i1 + 2 * q], p[8 * i1 + 2 * q + 1]);
            lsum[i1] = add_pair<E>(w[q], lsum[i1]);
          }
          pk[2 * nb + i1] = w;
        }
      }
    }
    lrun += lsum[0] + lsum[1];

    // O^T += V^T P^T; operand rows are d = 32db + pi(row), keys per slot as above
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int vb = ((db & 1) ? voff_odd : voff_even) + 64 * db;
#pragma unroll
      for (int u = 0; u < 2 * NB; ++u) {
        if (!MASKED || (u >> 1) < nvalid) {
          const int o = vb + 16 * u * ROWB;
          acc[db] = mfma32<E>(lds_read_tr16x2(Vs, o, o + 8 * ROWB), pk[u], acc[db]);
        }
      }
    }
  };

  auto step = [&](int j, auto par_tag, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool P = decltype(par_tag)::value;
    unsigned char* cur = P ? lds1 : lds0;
    unsigned char* nxt = P ? lds0 : lds1;
    if (j + 1 < ntiles) dma_tile(j + 1, nxt);
    compute(cur, j * BN, mask_tag);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
  };

  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();

  int j = 0;
  for (; j + 1 < jfull; j += 2) {
    step(j, Tag<false>{}, Tag<false>{});
    step(j + 1, Tag<true>{}, Tag<false>{});
  }
  if (j < jfull) {
    step(j, Tag<false>{}, Tag<false>{});
    ++j;
  }
  for (; j < ntiles; ++j) {
    if (j & 1) step(j, Tag<true>{}, Tag<true>{});
    else step(j, Tag<false>{}, Tag<true>{});
  }

  // ---- epilogue: O = acc / l; lane holds d = 32db + 16i1 + 8hh + 0..7
  const float ltot = halfwave_sum(lrun);
  const float inv = 1.0f / ltot;
  uint16_t* orow = O + qbase + (size_t)m * D;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int i1 = 0; i1 < 2; ++i1) {
      gstore16(orow + db * 32 + 16 * i1 + 8 * hh, pack8<E>(acc[db], 8 * i1, inv));
    }
  }
  if (LSE && hh == 0) Lse[(size_t)(b * H + hq) * S + m] = mrun + __log2f(ltot);
}

// ---------------------------------------------------------------------------
template <typename E, int D, int BM, int BN, int GH, bool LSE>
static int launch_fwd(const FwdArgs& a) {
  constexpr int NT = 64 * (BM / 32) * GH;
  const int total = a.B * (a.H / GH) * (a.S / BM);
  hipLaunchKernelGGL((fwd_kernel<E, D, BM, BN, GH, LSE>), dim3(total), dim3(NT), 0, (hipStream_t)a.stream,
                     (const uint16_t*)a.q, (const uint16_t*)a.k, (const uint16_t*)a.v,
                     (uint16_t*)a.o, a.lse, a.B, a.H, a.Hkv, a.S, a.scale_log2);
  return hipGetLastError() == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

// Dispatch over the compile-time parameters of one (element type, D) slice.
template <typename E, int D>
static FwdFn pick_fwd(int bm, int bn, int gh, bool lse) {
#define FA_CASE(BM_, BN_, GH_)                                                          \
  if (bm == BM_ && bn == BN_ && gh == GH_)                                             \
    return lse ? launch_fwd<E, D, BM_, BN_, GH_, true> : launch_fwd<E, D, BM_, BN_, GH_, false>;
  FA_CASE(64, 64, 1) FA_CASE(64, 128, 1) FA_CASE(128, 64, 1) FA_CASE(128, 128, 1)
  FA_CASE(64, 64, 2) FA_CASE(64, 128, 2) FA_CASE(128, 64, 2) FA_CASE(128, 128, 2)
  FA_CASE(64, 64, 4) FA_CASE(64, 128, 4)
#undef FA_CASE
  return nullptr;
}

}  // namespace fa

// FA_ETYPE (fa::F16 / fa::BF16), FA_D and FA_FWD_TABLE come from the build.
extern "C" FA_HIDDEN fa::FwdFn FA_FWD_TABLE(int bm, int bn, int gh, int lse) {
  return fa::pick_fwd<FA_ETYPE, FA_D>(bm, bn, gh, lse != 0);
}
