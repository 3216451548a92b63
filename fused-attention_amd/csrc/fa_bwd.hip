// fa_bwd.hip - atomic-free recompute backward of causal attention for gfx950.
//
// Math (attention/backward/fused_backward.py:66-147, report p.10 eq. 5), per (b, h):
//   P  = exp2(S*c - LSE)     with S = Q K^T, c = log2(e)/sqrt(D), LSE from the forward
//   dV = P^T dO              dP = dO V^T        Delta = rowsum(dO * O)
//   dS = P * (dP - Delta)    dQ = dS K / sqrt(D)  dK = dS^T Q / sqrt(D)
// Two kernels on the caller's stream: dK/dV then dQ, each forming Delta itself;
// or, given a buffer for per-row terms, dQ first (it writes each query row's
// -LSE/c and -Delta) and then dK/dV, which reads them instead of forming Delta.
//   dkdv_kernel: one workgroup per key tile (128 keys, 32 per wave) of one K/V
//                head; walks the (64-row query tile, query head) pairs at and below
//                the diagonal (G = H / Hkv heads per K/V head; 1 for MHA).  Per pair,
//                Q, dO, O and LSE (or Q, dO and the per-row terms) are copied
//                global -> LDS by DMA (triple buffered), and Delta is formed from
//                the O and dO tiles in LDS when not handed over.  Each wave keeps
//                its K and V rows in registers as MFMA B operands, computes S = Q K^T
//                and dP = dO V^T with one lane per key, and accumulates
//                dV^T += dO^T P and dK^T += Q^T dS, reading dO^T and Q^T with
//                ds_read_b64_tr_b16.  At D >= 64 the full tiles run a hand-pipelined
//                schedule (operand reads a region ahead of their MFMAs).
//   dkdv_pair_kernel: the same work at D = 128 when the per-row terms are handed
//                over, each 32-key block split over two waves by role (S, P and
//                dV / dP, dS and dK, P passed through LDS), so two waves share
//                every SIMD where dkdv_kernel fits one.
//   dkdv_reduce_kernel: only with a caller workspace, when B * H_kv key tiles alone
//                would leave the GPU idle (MQA, few heads): each key tile's pairs are
//                then split over several dK/dV workgroups that write fp32 partial
//                sums, and this pass adds them (fixed order) into dK and dV.
//   dq_kernel:   one workgroup per query tile (tile_m rows, 32 per wave); loops over
//                the key tiles (tile_n keys) up to the diagonal, heavy first.  Each
//                wave keeps Q and dO rows in registers, computes S^T = K Q^T and
//                dP^T = V dO^T with one lane per query (LSE and Delta are per-lane
//                scalars; Delta comes from the O and dO rows in the prologue, and is
//                stored with -LSE/c as the per-row terms when dK/dV runs after) and
//                accumulates dQ^T += K^T dS^T, reading K^T with transposed reads.
//                At D >= 64 the full tiles run a hand-pipelined schedule (operand
//                reads two items ahead of their MFMAs).
// No kernel uses atomics; each output element is written once.  Any S >= 1: the
// last query and key tiles may be partial (rows past S read as zero, never stored).
//
// LDS tiles are row-major with 16-byte chunk ch of row r stored at ch ^ bswz(r).
// gfx950's LDS has 64 banks of 4 bytes and serves a 16-byte read 16 lanes per
// cycle, an 8-byte read 16 lanes per cycle.  bswz makes both read kinds conflict
// free: 16 consecutive rows read at one chunk (an MFMA operand read) land on 16
// distinct 16-byte slots of the 256-byte bank line, and 4 consecutive rows read
// as one 32-byte piece (a transposed read) land on 4 distinct 32-byte groups.
#include <algorithm>
#include <type_traits>

#include "fa_device.h"
#include "fa_launch.h"

namespace fa {

typedef short i16x4b __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4b lds_i16x4b;

constexpr int kBwdWaitVmcnt0 = 0x0F70;  // s_waitcnt vmcnt(0)

// dK / dV at D = 128 with the row terms handed over: paired waves (1) or one wave
// per 32-key block (0)
#ifndef FA_DKDV_PAIR
#define FA_DKDV_PAIR 1
#endif

template <bool B>
struct BTag {
  static constexpr bool value = B;
};

template <int I>
using IC = std::integral_constant<int, I>;

// f(IC<I>{}) for I = I0 .. N-1, each with its index as a compile-time constant
template <int I0, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I0 < N) {
    f(IC<I0>{});
    static_for<I0 + 1, N>(f);
  }
}

// Chunk swizzle of row r for rows of cpr 16-byte chunks (cpr = 16, 8 or 4: rows
// of 256, 128 or 64 bytes, i.e. 1, 2 or 4 rows per bank line).
__host__ __device__ __forceinline__ int bswz(int r, int cpr) {
  if (cpr >= 16) return ((r & 3) << 1) | ((r >> 2) & 1) | (r & 8);
  if (cpr == 8) {
    const int k = r >> 1;
    return ((k & 3) << 1) | ((k >> 2) & 1);
  }
  return (r >> 2) & 3;
}

__device__ __forceinline__ u32x4 tr_read2(const unsigned char* base, int off0, int off1) {
  i16x4b a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4b*)(base + off0));
  i16x4b b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4b*)(base + off1));
  u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return u32x4{ua[0], ua[1], ub[0], ub[1]};
}

// Per-lane offsets into a swizzled row-major tile with rows of ROWB bytes.
//  opnd[t] (+ 32 qb * ROWB): MFMA operand read, lane c -> row c, chunk 2t + hh
//  tr(db, u, r2): transposed read feeding an A operand whose rows are
//    d = 32db + pi(lane % 32) and whose k-slots are rows 16u + 8*r2 + 4*hh + (0..3)
//    of the tile (the slot order of a score accumulator used as the B operand);
//    the swizzle of those rows depends only on (r2, hh, lane), not on u.
template <int ROWB>
struct TileOffsets {
  static constexpr int CPR = ROWB / 16, KT = ROWB / 32, DB = ROWB / 64;
  int opnd[KT];
  int trv[DB][2];
  __device__ __forceinline__ void init(int lane) {
    const int c = lane & 31, hh = lane >> 5;
#pragma unroll
    for (int t = 0; t < KT; ++t) opnd[t] = c * ROWB + (((2 * t + hh) ^ bswz(c, CPR)) << 4);
    const int G = lane >> 4, kr = (lane >> 2) & 3, c4 = lane & 3;
    const int b = 2 * pi_swap23(16 * (G & 1) + 4 * c4);   // byte offset of 4 d values in a 64-byte block
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int row = 8 * r2 + 4 * hh + kr;
      const int w = bswz(row, CPR);
#pragma unroll
      for (int db = 0; db < DB; ++db)
        trv[db][r2] = row * ROWB + ((((64 * db + b) >> 4) ^ w) << 4) + (b & 8);
    }
  }
  __device__ __forceinline__ int tr(int db, int u, int r2) const { return trv[db][r2] + 16 * u * ROWB; }
};

// Score-accumulator element (lane c, hh, register g) -> row offset inside a 32-row block.
__host__ __device__ __forceinline__ int acc_row(int g, int hh) { return 8 * (g >> 2) + 4 * hh + (g & 3); }

// ===========================================================================
// dK / dV
// ===========================================================================
// RB: the dQ kernel has already written each query row's -LSE/c and -Delta to
// Rb ([2, B*H, S]); the tiles then carry those 512 bytes instead of the O tile,
// and nothing is formed per tile.  Without RB each workgroup forms Delta from the
// O and dO tiles it stages (every key tile that meets a query tile repeats it).
template <typename E, int D, int BMQ, int BNK, bool RB>
__global__ __launch_bounds__(2 * BNK)
__attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1, D <= 64 ? 2 : 1)))
void dkdv_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                 const uint16_t* __restrict__ V, const uint16_t* __restrict__ O,
                 const uint16_t* __restrict__ dO, const float* __restrict__ Lse,
                 const float* __restrict__ Rb, uint16_t* __restrict__ dK, uint16_t* __restrict__ dV,
                 float* __restrict__ Pk, float* __restrict__ Pv, int nsplit,
                 int B, int H, int Hkv, int S, float scale_log2, float sm_scale) {
  static_assert(BMQ == 64, "a query tile is two 32-row blocks");
  constexpr int NW = BNK / 32;
  constexpr int NT = 64 * NW;
  constexpr int KT = D / 16, DB = D / 32;
  constexpr int ROWB = D * 2, CPR = ROWB / 16;
  constexpr int TILE = BMQ * ROWB;                       // bytes of one Q / dO / O tile
  constexpr int NBLK = TILE / 1024;
  // Q | dO | O | LSE, or with RB: Q | dO | -LSE/c | -Delta
  constexpr int OFF_L = (RB ? 2 : 3) * TILE;
  constexpr int BUFA = (OFF_L + (RB ? 2 : 1) * BMQ * 4 + 1023) / 1024 * 1024;
  constexpr int NBUF = 3;
  constexpr int TPR = NT / BMQ;                          // threads per row for Delta
  static_assert(TILE % 1024 == 0, "tiles are whole 1 KB DMA blocks");
  static_assert(TPR == 4 && (CPR % TPR) == 0, "Delta: one lane quad per row");
  const float NEG_INF = -__builtin_inff();

  // three tile buffers: tile i is computed while tile i+1 has landed (its Delta
  // is formed) and tile i+2 is in flight
  __shared__ __attribute__((aligned(1024))) unsigned char bufs[NBUF * BUFA];
  __shared__ __attribute__((aligned(16))) float delta_s[2][BMQ];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hh = lane >> 5;

  // work item: (b, K/V head, chunk, key tile), heaviest key tile (j = 0) first,
  // XCD aware.  A key tile meets T = G * NI (query tile, query head) pairs (G =
  // H / Hkv query heads per K/V head, 1 for MHA); with nsplit = 1 one workgroup
  // sums them all in its registers and writes dK and dV once, otherwise chunk c
  // takes pairs [T c / nsplit, T (c+1) / nsplit) and writes fp32 partial sums that
  // dkdv_reduce_kernel adds up.  The last key tile may be partial: waves whose keys
  // start past S stay inactive but still share the DMA and the barriers, and lanes
  // of keys past S are not stored.
  const int G = H / Hkv;
  const int nk = (S + BNK - 1) / BNK;
  const int total = B * Hkv * nsplit * nk;
  const int wg = blockIdx.x;
  const int L = (total % 8 == 0) ? (wg % 8) * (total / 8) + (wg / 8) : wg;
  const int u = L / nk, jt = L % nk;       // u = (b * Hkv + K/V head) * nsplit + chunk
  const int bkv = u / nsplit;              // b * Hkv + K/V head
  const size_t base = (size_t)bkv * S * D;
  const int bh0 = (bkv / Hkv) * H + (bkv % Hkv) * G;   // first query head of the group

  const int k0w = jt * BNK + 32 * wave;   // first key of this wave
  const int n = k0w + c;                  // this lane's key
  const bool active = k0w < S;            // wave-uniform

  // K, V rows as B operands: k-step t holds X[n][16t + 8hh .. +7]
  u32x4 kf[KT], vf[KT];
  if (active) {
    const uint16_t* kr = K + base + (size_t)min(n, S - 1) * D + 8 * hh;  // keys >= S: any valid row
    const uint16_t* vr = V + base + (size_t)min(n, S - 1) * D + 8 * hh;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      kf[t] = gload16(kr + 16 * t);
      vf[t] = gload16(vr + 16 * t);
    }
  }

  const int nq = (S + BMQ - 1) / BMQ;     // the last query tile may be partial
  const int i0 = (jt * BNK) / BMQ;        // first query tile that sees this key tile

  // DMA of the Q, dO and O tiles (row-major, swizzled) and the LSE slice of query
  // tile i into an LDS buffer: waves take 1 KB blocks round-robin and lane L of a
  // block writes LDS bytes blk*1024 + 16L.  Per-lane source offsets inside a tile
  // are fixed (dvo); each tile gets its own buffer descriptor.
  constexpr int NDMA = (NBLK + NW - 1) / NW;
  const int drow = lane / CPR, dch = lane % CPR;
  int dvo[NDMA];
#pragma unroll
  for (int x = 0; x < NDMA; ++x) {
    const int row = (wave + x * NW) * (1024 / ROWB) + drow;
    dvo[x] = row * ROWB + ((dch ^ bswz(row, CPR)) << 4);
  }
  // The workgroup walks its chunk of the (query tile, query head) pairs that meet
  // its keys in one sequence, query tile major: pair t = (i0 + t / G, t % G).
  // One sequence rather than a loop per head keeps the three-buffer pipeline full
  // across heads and leaves the tile loops un-nested.  Each tile's DMA uses
  // descriptors sized to the rows below S, so rows of a partial last query tile
  // read as zero (and contribute nothing: dO = 0 there).
  const int NI = nq - i0;                 // query tiles that meet this key tile (>= 1)
  const int T = G * NI;
  const int TE = G * min(2, NI);          // pairs on the two tiles that meet the keys
  const int hc = u % nsplit;
  const int tb = (int)((long long)T * hc / nsplit), te = (int)((long long)T * (hc + 1) / nsplit);
  // (the slot offset goes through readfirstlane as one scalar: left to itself the
  // compiler splits t % NBUF into two terms and adds both to every LDS address)
  auto bufp = [&](int t) __attribute__((always_inline)) {
    return bufs + __builtin_amdgcn_readfirstlane((t % NBUF) * BUFA);
  };
  int di = i0 + tb / G, dg = tb % G;      // the next pair to load, in sequence order
  auto dma_next = [&](unsigned char* buf) __attribute__((always_inline)) {
    const size_t row0 = (size_t)(bh0 + dg) * S + (size_t)di * BMQ;   // first row in [B, H, S]
    const int rows = min(BMQ, S - di * BMQ);
    const auto qrs = make_rsrc(Q + row0 * D, rows * ROWB);
    const auto dors = make_rsrc(dO + row0 * D, rows * ROWB);
#pragma unroll
    for (int x = 0; x < NDMA; ++x) {
      const int blk = wave + x * NW;
      if (NBLK % NW == 0 || blk < NBLK) {
        dma16(qrs, buf + blk * 1024, dvo[x], 0);
        dma16(dors, buf + TILE + blk * 1024, dvo[x], 0);
        if constexpr (!RB) dma16(make_rsrc(O + row0 * D, rows * ROWB), buf + 2 * TILE + blk * 1024, dvo[x], 0);
      }
    }
    if constexpr (RB) {
      if (wave == 0) dma4(make_rsrc(Rb + row0, rows * 4), buf + OFF_L, 4 * lane, 0);
      if (wave == 1) dma4(make_rsrc(Rb + (size_t)B * H * S + row0, rows * 4), buf + OFF_L + 4 * BMQ, 4 * lane, 0);
    } else {
      if (wave == 0) dma4(make_rsrc(Lse + row0, rows * 4), buf + OFF_L, 4 * lane, 0);
    }
    if (++dg == G) {
      dg = 0;
      ++di;
    }
  };

  TileOffsets<ROWB> to;
  to.init(lane);

  f32x16 dv_acc[DB], dk_acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dv_acc[db] = f32x16{};
    dk_acc[db] = f32x16{};
  }

  // Per tile, once: -Delta into dl (TPR threads per row, chunk subsets, shuffles)
  // and the tile's LSE slice rewritten in place as -LSE / c.  Both are then the
  // initial accumulators of the dP and S products, so the MFMAs deliver
  // dP - Delta and S - LSE/c directly.  With RB both arrive staged with the tile
  // and there is nothing to form.
  const float inv_c = 1.0f / scale_log2;
  auto delta_phase = [&](unsigned char* buf, float* dl) __attribute__((always_inline)) {
    if constexpr (RB) return;
    const int row = tid / TPR, part = tid % TPR;
    float acc = 0.f;
#pragma unroll
    for (int x = 0; x < CPR / TPR; ++x) {
      const int ch = part + TPR * x;
      const int off = row * ROWB + ((ch ^ bswz(row, CPR)) << 4);
      const u32x4 a = lds_read16(buf + TILE, off);
      const u32x4 o = lds_read16(buf + 2 * TILE, off);
#pragma unroll
      for (int w = 0; w < 4; ++w) acc = dot_pair<E>(a[w], o[w], acc);
    }
    acc = quad_sum(acc);
    // the four lanes of a row's quad store the same values (no branch, so this
    // joins the surrounding MFMA schedule)
    float* Ls = reinterpret_cast<float*>(buf + OFF_L);
    const float lsc = -Ls[row] * inv_c;
    dl[row] = -acc;
    Ls[row] = lsc;
  };

  // delta_phase in two steps, so the pipelined tile below can issue the reads a
  // region before the arithmetic
  auto delta_load = [&](const unsigned char* buf, u32x4 (&da)[CPR / TPR], u32x4 (&dob)[CPR / TPR], float& ls)
      __attribute__((always_inline)) {
    const int row = tid / TPR, part = tid % TPR;
#pragma unroll
    for (int x = 0; x < CPR / TPR; ++x) {
      const int off = row * ROWB + (((part + TPR * x) ^ bswz(row, CPR)) << 4);
      da[x] = lds_read16(buf + TILE, off);
      dob[x] = lds_read16(buf + 2 * TILE, off);
    }
    ls = reinterpret_cast<const float*>(buf + OFF_L)[row];
  };
  auto delta_store = [&](unsigned char* buf, float* dl, const u32x4 (&da)[CPR / TPR],
                         const u32x4 (&dob)[CPR / TPR], float ls) __attribute__((always_inline)) {
    const int row = tid / TPR;
    float acc = 0.f;
#pragma unroll
    for (int x = 0; x < CPR / TPR; ++x)
#pragma unroll
      for (int w = 0; w < 4; ++w) acc = dot_pair<E>(da[x][w], dob[x][w], acc);
    acc = quad_sum(acc);
    dl[row] = -acc;
    reinterpret_cast<float*>(buf + OFF_L)[row] = -ls * inv_c;
  };

  // Accumulator init for query block qb: register g <-> query row 32qb + acc_row(g),
  // i.e. four float4 runs at rows 32qb + 8gq + 4hh
  auto load_rows = [&](const float* src, int qb) __attribute__((always_inline)) {
    f32x16 v;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(src + 32 * qb + 8 * gq + 4 * hh);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * gq + e] = x[e];
    }
    return v;
  };

  // S - LSE/c = Q_b K^T - LSE/c and dP - Delta = dO_b V^T - Delta for 32-row query
  // block qb: lane (c = key, hh), register g -> query 32 qb + acc_row(g)
  auto sd = [&](const unsigned char* buf, const float* dl, int qb, f32x16& s, f32x16& dp) __attribute__((always_inline)) {
    s = load_rows(reinterpret_cast<const float*>(buf + OFF_L), qb);
    dp = load_rows(dl, qb);
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const int o = to.opnd[t] + 32 * qb * ROWB;
      s = mfma32<E>(lds_read16(buf, o), kf[t], s);
      dp = mfma32<E>(lds_read16(buf + TILE, o), vf[t], dp);
    }
  };
  // P = exp2(c (S - LSE/c)) and dS = P (dP - Delta), packed as B operands; on the
  // diagonal block keys past the query are masked
  auto grad = [&](int qb, const f32x16& s, const f32x16& dp, bool diag, u32x4 (&pk)[2], u32x4 (&dsk)[2])
      __attribute__((always_inline)) {
    float p[16], ds[16];
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      float x = s[g];
      if (diag && c > acc_row(g, hh)) x = NEG_INF;
      p[g] = fast_exp2(x * scale_log2);
      ds[g] = p[g] * dp[g];
    }
#pragma unroll
    for (int i1 = 0; i1 < 2; ++i1)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pk[i1][q] = pack2<E>(p[8 * i1 + 2 * q], p[8 * i1 + 2 * q + 1]);
        dsk[i1][q] = pack2<E>(ds[8 * i1 + 2 * q], ds[8 * i1 + 2 * q + 1]);
      }
  };
  // dV^T += dO^T P, dK^T += Q^T dS (k-slots: queries 32qb + 16i1 + 8r2 + 4hh + 0..3)
  auto wacc = [&](const unsigned char* buf, int qb, const u32x4 (&pk)[2], const u32x4 (&dsk)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) {
        const int u = 2 * qb + i1;
        dv_acc[db] = mfma32<E>(tr_read2(buf + TILE, to.tr(db, u, 0), to.tr(db, u, 1)), pk[i1], dv_acc[db]);
        dk_acc[db] = mfma32<E>(tr_read2(buf, to.tr(db, u, 0), to.tr(db, u, 1)), dsk[i1], dk_acc[db]);
      }
  };

  // a tile wholly past this wave's keys: both blocks in straight-line order so the
  // VALU of one block runs under the MFMAs of the other
  auto tile_full = [&](unsigned char* buf, const float* dl) __attribute__((always_inline)) {
    f32x16 s0, dp0, s1, dp1;
    u32x4 pk0[2], dsk0[2], pk1[2], dsk1[2];
    sd(buf, dl, 0, s0, dp0);
    sd(buf, dl, 1, s1, dp1);
    grad(0, s0, dp0, false, pk0, dsk0);
    wacc(buf, 0, pk0, dsk0);
    grad(1, s1, dp1, false, pk1, dsk1);
    wacc(buf, 1, pk1, dsk1);
  };

  // The same tile at D >= 64, as seven regions pinned by sched_barrier (at D = 128
  // one wave per SIMD, so nothing else hides its LDS latency; at D = 64 two): each
  // issues the operand reads of the next region's MFMAs while its own run, the P / dS math is spread
  // over four of them in halves, the reads of the next tile's Delta go out a region
  // before its arithmetic, and the last 8 dV/dK MFMAs (block 1, second half) move to
  // the first region of the next tile, where they cover the reads that follow its
  // barrier.  Same arithmetic in the same order as tile_full (bitwise equal); 12 %
  // faster at D = 128 (B=4 H=32 S=4096) than the compiler's own schedule, whose MFMAs
  // each waited for an operand read issued just before them, 3 % at D = 64.
  constexpr int KH = KT / 2, DH = DB / 2;
  auto rd_sd = [&](const unsigned char* buf, int qb, int half, u32x4 (&r)[2 * KH]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < KH; ++i) {
      const int o = to.opnd[KH * half + i] + 32 * qb * ROWB;
      r[i] = lds_read16(buf, o);
      r[KH + i] = lds_read16(buf + TILE, o);
    }
  };
  auto mm_sd = [&](int half, const u32x4 (&r)[2 * KH], f32x16& s, f32x16& dp) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < KH; ++i) {
      s = mfma32<E>(r[i], kf[KH * half + i], s);
      dp = mfma32<E>(r[KH + i], vf[KH * half + i], dp);
    }
  };
  auto rd_w = [&](const unsigned char* buf, int qb, int half, u32x4 (&r)[2 * KH]) __attribute__((always_inline)) {
    static_assert(D != 128 || 4 * DH == 2 * KH, "one operand buffer serves both phases");
#pragma unroll
    for (int j = 0; j < DH; ++j)
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) {
        const int db = DH * half + j, u = 2 * qb + i1;
        r[2 * (2 * j + i1)] = tr_read2(buf + TILE, to.tr(db, u, 0), to.tr(db, u, 1));
        r[2 * (2 * j + i1) + 1] = tr_read2(buf, to.tr(db, u, 0), to.tr(db, u, 1));
      }
  };
  auto mm_w = [&](int half, const u32x4 (&r)[2 * KH], const u32x4 (&pk)[2], const u32x4 (&dsk)[2])
      __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < DH; ++j)
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) {
        const int db = DH * half + j;
        dv_acc[db] = mfma32<E>(r[2 * (2 * j + i1)], pk[i1], dv_acc[db]);
        dk_acc[db] = mfma32<E>(r[2 * (2 * j + i1) + 1], dsk[i1], dk_acc[db]);
      }
  };
  // P and dS of one half (registers 8 i1 .. 8 i1 + 7) of an unmasked block
  auto grad_half = [&](int i1, const f32x16& s, const f32x16& dp, u32x4 (&pk)[2], u32x4 (&dsk)[2])
      __attribute__((always_inline)) {
    float p[8], ds[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      p[g] = fast_exp2(s[8 * i1 + g] * scale_log2);
      ds[g] = p[g] * dp[8 * i1 + g];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pk[i1][q] = pack2<E>(p[2 * q], p[2 * q + 1]);
      dsk[i1][q] = pack2<E>(ds[2 * q], ds[2 * q + 1]);
    }
  };
  u32x4 c_r[2 * KH], c_pk[2], c_dsk[2];   // the deferred MFMAs' operands
  auto tile_full_pipelined = [&](unsigned char* buf, const float* dl, unsigned char* nbuf, float* ndl, auto prev)
      __attribute__((always_inline)) {
    f32x16 s0, dp0, s1, dp1;
    u32x4 pk0[2], dsk0[2], pk1[2], dsk1[2];
    u32x4 ra[2 * KH], rb[2 * KH];
    const float* lse_s = reinterpret_cast<const float*>(buf + OFF_L);
    s0 = load_rows(lse_s, 0);
    dp0 = load_rows(dl, 0);
    rd_sd(buf, 0, 0, ra);
    if constexpr (decltype(prev)::value) mm_w(1, c_r, c_pk, c_dsk);   // the previous tile's last MFMAs
    __builtin_amdgcn_sched_barrier(0);
    rd_sd(buf, 0, 1, rb);
    mm_sd(0, ra, s0, dp0);
    s1 = load_rows(lse_s, 1);
    dp1 = load_rows(dl, 1);
    __builtin_amdgcn_sched_barrier(0);
    rd_sd(buf, 1, 0, ra);
    mm_sd(1, rb, s0, dp0);
    __builtin_amdgcn_sched_barrier(0);
    rd_sd(buf, 1, 1, rb);
    mm_sd(0, ra, s1, dp1);
    grad_half(0, s0, dp0, pk0, dsk0);
    __builtin_amdgcn_sched_barrier(0);
    rd_w(buf, 0, 0, ra);
    mm_sd(1, rb, s1, dp1);
    grad_half(1, s0, dp0, pk0, dsk0);
    __builtin_amdgcn_sched_barrier(0);
    rd_w(buf, 0, 1, rb);
    mm_w(0, ra, pk0, dsk0);
    grad_half(0, s1, dp1, pk1, dsk1);
    __builtin_amdgcn_sched_barrier(0);
    rd_w(buf, 1, 0, ra);
    mm_w(1, rb, pk0, dsk0);
    grad_half(1, s1, dp1, pk1, dsk1);
    u32x4 da[CPR / TPR], dob[CPR / TPR];
    float ls;
    if constexpr (!RB) delta_load(nbuf, da, dob, ls);
    __builtin_amdgcn_sched_barrier(0);
    rd_w(buf, 1, 1, c_r);
    mm_w(0, ra, pk1, dsk1);
    if constexpr (!RB) delta_store(nbuf, ndl, da, dob, ls);
#pragma unroll
    for (int i1 = 0; i1 < 2; ++i1) {
      c_pk[i1] = pk1[i1];
      c_dsk[i1] = dsk1[i1];
    }
  };
  // a tile meeting this wave's keys: blocks before the keys are skipped (always,
  // for an inactive wave), the block starting at the wave's first key is masked
  // (a rolled loop: it runs for two tiles per workgroup, and unrolling it would
  // merge both blocks' live state into one schedule)
  auto tile_edge = [&](unsigned char* buf, const float* dl, int qtile0) __attribute__((always_inline)) {
#pragma nounroll
    for (int qb = 0; qb < 2; ++qb) {
      const int qrow0 = qtile0 + 32 * qb;
      if (qrow0 + 31 < k0w) continue;
      f32x16 s, dp;
      u32x4 pk[2], dsk[2];
      sd(buf, dl, qb, s, dp);
      grad(qb, s, dp, qrow0 == k0w, pk, dsk);
      wacc(buf, qb, pk, dsk);
    }
  };

  // ---- main loop over the pairs: at the top of iteration t pair t+1 has landed
  // (one barrier makes it and Delta(t) visible), pair t+2 starts its DMA into the
  // buffer pair t-1 used, pair t is computed, Delta(t+1) formed
  // where pair t's -Delta rows are: formed into delta_s, or staged with the tile
  auto dlp = [&](int t) __attribute__((always_inline)) -> float* {
    if constexpr (RB) return reinterpret_cast<float*>(bufp(t) + OFF_L + 4 * BMQ);
    else return delta_s[t & 1];
  };
  auto top = [&](int t) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
    __syncthreads();
    if (t + 2 < te) dma_next(bufp(t + 2));
  };
  auto bottom = [&](int t) __attribute__((always_inline)) {
    if (t + 1 < te) delta_phase(bufp(t + 1), dlp(t + 1));
  };
  if (tb < te) {  // (a chunk of a light key tile can be empty: it stores zeros)
    dma_next(bufp(tb));
    if (tb + 1 < te) dma_next(bufp(tb + 1));
    __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
    __syncthreads();
    delta_phase(bufp(tb), dlp(tb));
  }
  // the pairs on the two tiles that meet this workgroup's keys, then the full tiles
  // (one straight path per loop keeps the accumulators in place across iterations)
  int t = tb;
  for (; t < min(te, TE); ++t) {
    top(t);
    tile_edge(bufp(t), dlp(t), (i0 + (t >= G ? 1 : 0)) * BMQ);
    bottom(t);
  }
  if (active) {
    // Delta(t+1) is formed first, in the same schedule as pair t's MFMAs; after
    // the last pair it runs on the idle buffer and its result is never read
    if constexpr (D >= 64) {
      // top(t) and the tile in one scope whose three buffers are restrict-qualified:
      // the compiler then knows the DMA into pair t+2's buffer cannot touch the
      // tiles being read, and drops the wait for that DMA it otherwise puts before
      // the first transposed read of every tile (2 % of the kernel)
      auto step = [&](int t, unsigned char* __restrict__ cur, unsigned char* __restrict__ nxt,
                      unsigned char* __restrict__ dst, auto prev) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
        __syncthreads();
        if (t + 2 < te) dma_next(dst);
        float* dl_c = RB ? reinterpret_cast<float*>(cur + OFF_L + 4 * BMQ) : delta_s[t & 1];
        float* dl_n = RB ? reinterpret_cast<float*>(nxt + OFF_L + 4 * BMQ) : delta_s[(t + 1) & 1];
        tile_full_pipelined(cur, dl_c, nxt, dl_n, prev);
      };
      if (t < te) {
        step(t, bufp(t), bufp(t + 1), bufp(t + 2), BTag<false>{});
        for (++t; t < te; ++t) step(t, bufp(t), bufp(t + 1), bufp(t + 2), BTag<true>{});
        mm_w(1, c_r, c_pk, c_dsk);
      }
    } else {
      for (; t < te; ++t) {
        top(t);
        delta_phase(bufp(t + 1), dlp(t + 1));
        tile_full(bufp(t), dlp(t));
      }
    }
  } else {
    for (; t < te; ++t) {
      top(t);
      bottom(t);
    }
  }

  // ---- epilogue: lane holds key n, d = 32db + 16i1 + 8hh + 0..7
  if (!active || n >= S) return;
  if (nsplit > 1) {  // fp32 partial sums of this chunk, dK already scaled
    float* pkr = Pk + ((size_t)u * S + n) * D;
    float* pvr = Pv + ((size_t)u * S + n) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) {
        const int d0 = db * 32 + 16 * i1 + 8 * hh;
#pragma unroll
        for (int h4 = 0; h4 < 2; ++h4) {
          const int g0 = 8 * i1 + 4 * h4;
          gstore_f32x4(pkr + d0 + 4 * h4, f32x4{dk_acc[db][g0] * sm_scale, dk_acc[db][g0 + 1] * sm_scale,
                                                dk_acc[db][g0 + 2] * sm_scale, dk_acc[db][g0 + 3] * sm_scale});
          gstore_f32x4(pvr + d0 + 4 * h4, f32x4{dv_acc[db][g0], dv_acc[db][g0 + 1], dv_acc[db][g0 + 2], dv_acc[db][g0 + 3]});
        }
      }
    }
    return;
  }
  uint16_t* dkr = dK + base + (size_t)n * D;
  uint16_t* dvr = dV + base + (size_t)n * D;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int i1 = 0; i1 < 2; ++i1) {
      gstore16(dkr + db * 32 + 16 * i1 + 8 * hh, pack8<E>(dk_acc[db], 8 * i1, sm_scale));
      gstore16(dvr + db * 32 + 16 * i1 + 8 * hh, pack8<E>(dv_acc[db], 8 * i1, 1.0f));
    }
  }
}

// ===========================================================================
// dK / dV with paired waves (D = 128, per-row terms handed over)
// ===========================================================================
// The work items, pair sequence and DMA of dkdv_kernel<..., RB = true>, with
// each 32-key block split over two waves by role instead of one wave holding
// everything:
//   role 0 keeps the K rows and dV:  S = Q_b K^T - LSE/c,  P = exp2(c S),
//          dV^T += dO^T P;  it leaves P in LDS for its partner as fp16 (P lies
//          in [0, 1]: fp16's 11-bit significand keeps the rounding of P 8x below
//          bf16's, and fp32 slots would not fit beside the three tile buffers)
//   role 1 keeps the V rows and dK:  dP = dO_b V^T - Delta,  dS = P dP,
//          dK^T += Q^T dS, with P read back from LDS.
// Each wave needs about half the registers of a dkdv_kernel wave (one K or V
// row set and one accumulator instead of two of each), so two waves share every
// SIMD, one of each role, and each one's LDS and MFMA latencies run under the
// other's work; dkdv_kernel at D = 128 holds one wave per SIMD.  The roles run
// a pair apart in one loop with one barrier per pair: in iteration t role 0
// forms S and P of pair t+1, then adds pair t to dV (P(t) kept packed in
// registers); role 1 adds pair t to dK (P(t) from LDS, dP(t) kept from the
// previous iteration), then forms dP of pair t+1.  Each SIMD thus mixes the
// full-rate operand reads of one product with the transposed reads of the
// other throughout the iteration.  P of pair t sits in slot t % 2.  The grid holds
// one workgroup per CU, each walking a fixed share of the key tiles (see the work
// items below) with the next tile's first pairs loaded under the current one's last.
template <typename E, int D, int BMQ, int BNK>
__global__ __launch_bounds__(4 * BNK)
__attribute__((amdgpu_waves_per_eu(2, 2)))
void dkdv_pair_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                      const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO,
                      const float* __restrict__ Rb, uint16_t* __restrict__ dK, uint16_t* __restrict__ dV,
                      float* __restrict__ Pk, float* __restrict__ Pv, int nsplit,
                      int B, int H, int Hkv, int S, float scale_log2, float sm_scale) {
  static_assert(BMQ == 64, "a query tile is two 32-row blocks");
  constexpr int NKB = BNK / 32;                          // key blocks = wave pairs
  constexpr int NW = 2 * NKB;
  constexpr int KT = D / 16, DB = D / 32;
  constexpr int ROWB = D * 2, CPR = ROWB / 16;
  constexpr int TILE = BMQ * ROWB;                       // bytes of one Q / dO tile
  constexpr int NBLK = TILE / 1024;
  constexpr int OFF_L = 2 * TILE;                        // Q | dO | -LSE/c | -Delta
  constexpr int BUFA = (OFF_L + 2 * BMQ * 4 + 1023) / 1024 * 1024;
  constexpr int NBUF = 3;
  // DMA waves: the four of role 0, whose stream is the shorter one (against all eight
  // waves: +1.6 % and +2.2 % at GQA B=2 H=32 H_kv=8 S=4096 and B=1 H=32 H_kv=4 S=8192, +0.9 %
  // at MHA B=4 H=32 S=4096; the same split on the upward walk, the kernel's earlier form,
  // lost 1.2 % there)
  constexpr int NDW = NW / 2;
  constexpr int NDMA = NBLK / NDW;
  constexpr int XPS = NKB * 2 * 2 * 64;                  // 16-byte P pieces per slot
  static_assert(TILE % 1024 == 0 && NBLK % NW == 0, "tiles are whole 1 KB DMA blocks, split evenly");
  const float NEG_INF = -__builtin_inff();

  __shared__ __attribute__((aligned(1024))) unsigned char bufs[NBUF * BUFA];
  // the P handed over: fp16 pairs (the same words as the dV operand for fp16 input)
  constexpr bool PF16 = std::is_same<E, F16>::value;
  // packed P, two slots: piece (query block qb, k-step half i1) of lane L of key
  // block kb at [slot][kb][qb][i1][L] (each wave's 16-byte write or read is 1 KB
  // contiguous)
  __shared__ __attribute__((aligned(16))) u32x4 xp[2 * XPS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int role = wave / NKB, kb = wave % NKB;
  const int c = lane & 31, hh = lane >> 5;

  // ---- work items: key tile jt of chunk hc of K/V head bkv (u = bkv nsplit + hc),
  // L = u nk + jt, the items of XCD x either the range [x total/8, (x+1) total/8) or
  // (total not a multiple of 8) L = 8i + x; within a head the heaviest key tiles
  // come first.  The grid holds only the workgroups that run at once (one per CU):
  // slot wg / 8 of XCD wg % 8 takes its XCD's items in rounds of gridDim.x / 8 items,
  // mirrored in odd rounds, so a heavy key tile and a light one pair up.  While an
  // item's last two pairs run, the next item's first two pairs and its K/V rows are
  // loaded (a workgroup's start-up, ~6 us of a ~57 us item at B=4 H=32 S=4096 D=128,
  // otherwise leaves its CU idle).
  // An item's pairs: the key tile's walk index w = G (di - i0) + dg covers query tiles
  // di >= i0 (its diagonal tile) of the G query heads bh0 + dg; of the T = G (nq - i0)
  // indices, chunk hc takes the w with w % nsplit == hc.  The walk alternates: items
  // of even rounds run their chunk from the last query tile down, odd rounds from the
  // diagonal up (an upward walk of contiguous chunks, its earlier form, read each Q/dO
  // tile once per key tile where a K/V head's G heads of Q and dO exceed the L2, and
  // measured at or below this one everywhere): the slots of an XCD all start an even round at the last query tile,
  // and each starts its odd-round item (diagonal two tiles below where its even-round
  // item ended) at the time the others pass that tile, so the XCD's workgroups read
  // the same Q/dO tiles at about the same time and each is fetched about once, not
  // once per key tile.
  const int G = H / Hkv;
  const int nk = (S + BNK - 1) / BNK;
  const int total = B * Hkv * nsplit * nk;
  const int nq = (S + BMQ - 1) / BMQ;
  const int wg = blockIdx.x;
  const int slots = (int)gridDim.x / 8, my_slot = wg / 8, xcd = wg % 8;
  auto item_L = [&](int k) __attribute__((always_inline)) {  // -1: no k-th item
    const int i = k * slots + ((k & 1) ? slots - 1 - my_slot : my_slot);
    if (total % 8 == 0) return i < total / 8 ? xcd * (total / 8) + i : -1;
    const int L = 8 * i + xcd;
    return L < total ? L : -1;
  };
  struct KItem {
    int u, jt, bh0, i0, hc, rev, tb, te;
    size_t base;
  };
  auto make_item = [&](int L, int k) __attribute__((always_inline)) {
    KItem it;
    it.u = L / nk;
    it.jt = L % nk;
    const int bkv = it.u / nsplit;
    it.base = (size_t)bkv * S * D;
    it.bh0 = (bkv / Hkv) * H + (bkv % Hkv) * G;
    it.i0 = (it.jt * BNK) / BMQ;
    const int T = G * (nq - it.i0), hc = it.u % nsplit;
    it.hc = hc;
    it.rev = (k & 1) ? 0 : 1;
    it.tb = 0;
    it.te = T > hc ? (T - hc + nsplit - 1) / nsplit : 0;
    return it;
  };
  const int L0 = item_L(0);
  if (L0 < 0) return;  // the grid is rounded up to a multiple of 8

  // the current item, as the code below reads it, and the next one (plain scalars:
  // as structs chosen at run time they went to scratch memory)
  // an item's sequence runs over positions tb .. te-1 (tb = 0)
  int u, jt, bh0, i0, hc, rev, tb, te, k0w, n;
  size_t base;
  bool active;
  int n_u = 0, n_jt = 0, n_bh0 = 0, n_i0 = 0, n_hc = 0, n_rev = 0, n_tb = 0, n_te = 0;
  size_t n_base = 0;
  bool has_next = false;
  auto set_item = [&](const KItem& it) __attribute__((always_inline)) {
    u = it.u;
    jt = it.jt;
    bh0 = it.bh0;
    i0 = it.i0;
    hc = it.hc;
    rev = it.rev;
    tb = it.tb;
    te = it.te;
    base = it.base;
    k0w = jt * BNK + 32 * kb;   // first key of this wave's block
    n = k0w + c;                // this lane's key
    active = k0w < S;           // wave-uniform
  };
  set_item(make_item(L0, 0));

  // K (role 0) or V (role 1) rows as B operands: k-step t holds X[n][16t + 8hh .. +7]
  u32x4 xf[KT];
  auto load_xf = [&](int xjt, size_t xbase) __attribute__((always_inline)) {
    const int kw = xjt * BNK + 32 * kb;
    if (kw < S) {
      const uint16_t* xr = (role ? V : K) + xbase + (size_t)min(kw + c, S - 1) * D + 8 * hh;
#pragma unroll
      for (int t = 0; t < KT; ++t) xf[t] = gload16(xr + 16 * t);
    }
  };

  // DMA of pair (di, dg)'s Q and dO tiles and its two row-term slices: each DMA wave
  // copies NDMA 1 KB blocks of each tile, waves 0 and 1 one slice each
  const int drow = lane / CPR, dch = lane % CPR;
  int dvo[NDMA];
#pragma unroll
  for (int x = 0; x < NDMA; ++x) {
    const int row = (wave % NDW + x * NDW) * (1024 / ROWB) + drow;
    dvo[x] = row * ROWB + ((dch ^ bswz(row, CPR)) << 4);
  }
  // pair p of the current item sits in buffer (p + boff) % NBUF; boff carries the
  // rotation into the next item (whose first pairs are loaded during this one)
  int boff = 0;
  auto bufp = [&](int t) __attribute__((always_inline)) {
    return bufs + __builtin_amdgcn_readfirstlane(((t + boff) % NBUF) * BUFA);
  };
  // position p of an item (chunk ihc, direction irev, positions 0 .. ite-1): walk
  // index w, i.e. query tile i0 + w / G of query head bh0 + w % G
  auto walk_w = [&](int p, int ihc, int irev, int ite) __attribute__((always_inline)) {
    return ihc + (irev ? ite - 1 - p : p) * nsplit;
  };
  auto qtile = [&](int p) __attribute__((always_inline)) { return i0 + walk_w(p, hc, rev, te) / G; };
  // the pair's DMA in 2 NDMA + 1 parts: part 2x / 2x+1 = block x of the Q / dO tile,
  // part 2 NDMA = the row-term slice (waves 0 and 1)
  struct Dma {
    __amdgpu_buffer_rsrc_t q, d, r;
    unsigned char* buf;
  };
  auto dma_prep = [&](int dbh, int qi0, int w, unsigned char* buf) __attribute__((always_inline)) {
    const int di = qi0 + w / G, dg = w % G;
    const size_t row0 = (size_t)(dbh + dg) * S + (size_t)di * BMQ;
    const int rows = min(BMQ, S - di * BMQ);
    Dma j{make_rsrc(Q + row0 * D, rows * ROWB), make_rsrc(dO + row0 * D, rows * ROWB),
          make_rsrc(Rb + (wave == 1 ? (size_t)B * H * S : 0) + row0, rows * 4), buf};
    return j;
  };
  // the pair at position p of the current item's sequence, continued into the next
  // item's first two pairs (false: none): walk index w of the item with query heads
  // from dbh and diagonal tile qi0
  auto dma_at = [&](int p, int& dbh, int& qi0, int& w) __attribute__((always_inline)) {
    if (p < te) {
      dbh = bh0;
      qi0 = i0;
      w = walk_w(p, hc, rev, te);
      return true;
    }
    if (!has_next) return false;
    dbh = n_bh0;
    qi0 = n_i0;
    const int pp = n_tb + (p - te);
    w = walk_w(pp, n_hc, n_rev, n_te);
    return pp < n_te;
  };
  auto dma_part = [&](const Dma& j, int k) __attribute__((always_inline)) {
    if (k < 2 * NDMA) {
      if (wave < NDW) {
        const int blk = wave + (k >> 1) * NDW;
        dma16((k & 1) ? j.d : j.q, j.buf + (k & 1) * TILE + blk * 1024, dvo[k >> 1], 0);
      }
    } else if (wave < 2) {
      dma4(j.r, j.buf + OFF_L + wave * 4 * BMQ, 4 * lane, 0);
    }
  };
  auto dma_pair = [&](int dbh, int qi0, int w, unsigned char* buf) __attribute__((always_inline)) {
    const Dma j = dma_prep(dbh, qi0, w, buf);
#pragma unroll
    for (int k = 0; k <= 2 * NDMA; ++k) dma_part(j, k);
  };

  TileOffsets<ROWB> to;
  to.init(lane);

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

  const int a1 = role ? TILE : 0;               // S / dP A rows: Q or dO
  const int a2 = role ? 0 : TILE;               // dV / dK A^T rows: dO or Q
  const int lo = OFF_L + role * 4 * BMQ;        // -LSE/c or -Delta
  auto slot = [&](int t, int qb, int i1) __attribute__((always_inline)) {
    return xp + (t & 1) * XPS + ((kb * 2 + qb) * 2 + i1) * 64 + lane;
  };

  auto load_rows = [&](const float* src, int qb) __attribute__((always_inline)) {
    f32x16 v;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(src + 32 * qb + 8 * gq + 4 * hh);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * gq + e] = x[e];
    }
    return v;
  };
  // query block qb of pair t meets this wave's keys (wave-uniform)
  auto live = [&](int t, int qb) __attribute__((always_inline)) {
    return active && qtile(t) * BMQ + 32 * qb + 31 >= k0w;
  };

  // front(t): S - LSE/c (role 0) or dP - Delta (role 1) of pair t's two query
  // blocks, the blocks' MFMA chains interleaved; role 0 turns S into P (keys past
  // the query masked on the diagonal block), keeps it packed in pk and writes it to
  // slot t % 2.  FULL: pair t lies wholly past this wave's keys (no test, no mask).
  auto front = [&](int t, f32x16 (&x)[2], u32x4 (&pk)[2][2], auto full) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full)::value;
    const unsigned char* buf = bufp(t);
    const int qrow0 = qtile(t) * BMQ;
    const bool l0 = FULL || live(t, 0), l1 = FULL || live(t, 1);
    if (!l1) return;  // (l0 implies l1)
    x[1] = load_rows(reinterpret_cast<const float*>(buf + lo), 1);
    if (l0) {
      x[0] = load_rows(reinterpret_cast<const float*>(buf + lo), 0);
#pragma unroll
      for (int t2 = 0; t2 < KT; ++t2) {
        x[0] = mfma32<E>(lds_read16(buf + a1, to.opnd[t2]), xf[t2], x[0]);
        x[1] = mfma32<E>(lds_read16(buf + a1, to.opnd[t2] + 32 * ROWB), xf[t2], x[1]);
      }
    } else {
#pragma unroll
      for (int t2 = 0; t2 < KT; ++t2)
        x[1] = mfma32<E>(lds_read16(buf + a1, to.opnd[t2] + 32 * ROWB), xf[t2], x[1]);
    }
    if (role != 0) return;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      if (qb == 0 && !l0) continue;
      const bool diag = !FULL && qrow0 + 32 * qb == k0w;
      float p[16];
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        float v = x[qb][g];
        if (diag && c > acc_row(g, hh)) v = NEG_INF;
        p[g] = fast_exp2(v * scale_log2);
      }
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) {
        u32x4 h;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          pk[qb][i1][q] = pack2<E>(p[8 * i1 + 2 * q], p[8 * i1 + 2 * q + 1]);
          h[q] = PF16 ? pk[qb][i1][q] : pack2<F16>(p[8 * i1 + 2 * q], p[8 * i1 + 2 * q + 1]);
        }
        *slot(t, qb, i1) = h;
      }
    }
  };
  // back(t): dV^T += dO^T P (role 0, P from pk) or dK^T += Q^T dS with
  // dS = P (dP - Delta) (role 1, P from slot t % 2, dP - Delta from x); k-slots:
  // queries 32qb + 16i1 + 8r2 + 4hh + 0..3
  auto back = [&](int t, const f32x16 (&x)[2], const u32x4 (&pk)[2][2], auto full) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full)::value;
    const unsigned char* buf = bufp(t);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      if (!FULL && !live(t, qb)) continue;
      u32x4 bop[2];
      if (role == 0) {
        bop[0] = pk[qb][0];
        bop[1] = pk[qb][1];
      } else {
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) {
          const u32x4 w = *slot(t, qb, i1);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int g = 8 * i1 + 2 * q;
            bop[i1][q] = pack2<E>(mul_f16_f32<0>(w[q], x[qb][g]), mul_f16_f32<1>(w[q], x[qb][g + 1]));
          }
        }
      }
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) {
          const int uu = 2 * qb + i1;
          acc[db] = mfma32<E>(tr_read2(buf + a2, to.tr(db, uu, 0), to.tr(db, uu, 1)), bop[i1], acc[db]);
        }
    }
  };

  // positions [tb, E0) and [E1, te) hold the pairs of query tiles i0 and i0 + 1, which
  // meet this workgroup's keys (edge tests, the diagonal mask); [max(tb, E0), E1) lie
  // wholly past them.  Only the last key tile can have inactive waves, and it meets at most
  // two query tiles (NI <= 2), so the full paths need no activity test.
  int E0 = 0, E1 = 0;
  auto set_edges = [&]() __attribute__((always_inline)) {
    const int TEw = G * min(2, nq - i0);                // walk indices of the edge pairs
    const int ne = TEw > hc ? (TEw - hc + nsplit - 1) / nsplit : 0;
    E0 = rev ? 0 : ne;
    E1 = rev ? te - ne : te;
  };
  // pair t+1 has landed, P(t) is visible, and nobody reads pair t-1's buffer or
  // slot (t+1) % 2 any more
  auto sync = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
    __syncthreads();
  };
  auto top = [&](int t) __attribute__((always_inline)) {
    sync();
    int dbh, dqi, dpp;
    if (dma_at(t + 2, dbh, dqi, dpp)) dma_pair(dbh, dqi, dpp, bufp(t + 2));
    // the item's last pair: its K/V rows are used no more, the next item's load
    if (t == te - 1 && has_next) load_xf(n_jt, n_base);
  };
  f32x16 x[2];
  u32x4 pk[2][2], pkn[2][2];
  // the item's first pairs (those not loaded during the previous item), then S / dP
  // of its first pair
  int pre = 0;        // bit i: pair tb + i of this item already in flight
  bool xf_pre = false;
  bool first = true;
  // ---- epilogue: lane holds key n, d = 32db + 16i1 + 8hh + 0..7; role 0 stores
  // dV, role 1 dK (keys past S: nothing)
  auto epilogue = [&]() __attribute__((always_inline)) {
    if (!active || n >= S) return;
    const float mul = role ? sm_scale : 1.0f;
    if (nsplit > 1) {  // fp32 partial sums of this chunk, dK already scaled
      float* pr = (role ? Pk : Pv) + ((size_t)u * S + n) * D;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) {
          const int d0 = db * 32 + 16 * i1 + 8 * hh;
#pragma unroll
          for (int h4 = 0; h4 < 2; ++h4) {
            const int g0 = 8 * i1 + 4 * h4;
            gstore_f32x4(pr + d0 + 4 * h4, f32x4{acc[db][g0] * mul, acc[db][g0 + 1] * mul,
                                                 acc[db][g0 + 2] * mul, acc[db][g0 + 3] * mul});
          }
        }
      return;
    }
    uint16_t* r = (role ? dK : dV) + base + (size_t)n * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) gstore16(r + db * 32 + 16 * i1 + 8 * hh, pack8<E>(acc[db], 8 * i1, mul));
  };
  auto prologue = [&]() __attribute__((always_inline)) {
    if (!xf_pre) load_xf(jt, base);
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
    if (tb >= te) return;  // (a chunk of a light key tile can be empty: it stores zeros)
    if (!(pre & 1)) dma_pair(bh0, i0, walk_w(tb, hc, rev, te), bufp(tb));
    if (tb + 1 < te && !(pre & 2)) dma_pair(bh0, i0, walk_w(tb + 1, hc, rev, te), bufp(tb + 1));
    if (first && tb + 1 < te) {
      // pair tb has landed once at most pair tb+1's operations are outstanding
      if (wave >= NDW) __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);  // (no DMA of its own)
      else if (wave < 2) __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0 | (2 * NDMA + 1));
      else __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0 | (2 * NDMA));
    } else {
      __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
    }
    __syncthreads();
    if (tb >= E0 && tb < E1) front(tb, x, pk, BTag<true>{});
    else front(tb, x, pk, BTag<false>{});
  };
  // Full pairs with a next pair run as one stream of 32 MFMAs per wave, operand
  // reads issued three MFMAs ahead (a rotating set of four, pinned by
  // sched_barrier; left to itself the compiler issued each read just before its
  // MFMA and waited on it):
  //   role 0: S(t+1) (full-rate reads; both query blocks' chains interleaved),
  //           then dV(t) (transposed reads), with P(t+1) formed, packed and
  //           written to its slot under the dV MFMAs
  //   role 1: dK(t) (transposed reads), with dS(t) formed from slot t % 2 and x
  //           first, then dP(t+1) (full-rate reads) into x
  // so the two waves of a SIMD read LDS at full and at half rate in turn.  A
  // dV / dK MFMA j = 0..15 is (query block j / 8, d block (j / 2) % 4, k-step
  // half j % 2), so every accumulator sees its products in the order back() adds
  // them; an S / dP MFMA j is k-step j / 2 of query block j % 2.
  auto rd_sd = [&](const unsigned char* buf, int j) __attribute__((always_inline)) {
    return lds_read16(buf + a1, to.opnd[j >> 1] + 32 * (j & 1) * ROWB);
  };
  // S / dP and dV / dK MFMAs per wave and pair: 2 KT and 4 DB (16 and 16 at D = 128)
  constexpr int NS = 2 * KT, NV = 4 * DB, NT = NS + NV;
  auto rd_w = [&](const unsigned char* buf, int j) __attribute__((always_inline)) {
    const int qb = j / (2 * DB), db = (j >> 1) % DB, i1 = j & 1;
    return tr_read2(buf + a2, to.tr(db, 2 * qb + i1, 0), to.tr(db, 2 * qb + i1, 1));
  };
  // A stream also issues pair t+2's DMA.  The source places one part every other
  // MFMA from the first, but the parts' run-time tests (pair t+2 may not exist) are
  // merged by the compiler into one block at the top of the stream, so the whole
  // DMA goes out right after the barrier, its descriptors formed first.  Measured,
  // that is the better place: with the parts pinned where the source puts them
  // (the test made compile-time), the backward ran 2.0 % slower at B=4 H=32 S=4096
  // D=128 and 8.1 % slower at GQA B=2 H=32 H_kv=8 S=4096: a part issued later has
  // less of the stream to land in.
  auto stream0 = [&](int t, const u32x4 (&pcur)[2][2], u32x4 (&pnxt)[2][2]) __attribute__((always_inline)) {
    int dbh, dqi, dpp;
    const bool dm = dma_at(t + 2, dbh, dqi, dpp);
    Dma job;
    if (dm) job = dma_prep(dbh, dqi, dpp, bufp(t + 2));
    const unsigned char* bn = bufp(t + 1);
    const unsigned char* bc = bufp(t);
    x[0] = load_rows(reinterpret_cast<const float*>(bn + lo), 0);
    x[1] = load_rows(reinterpret_cast<const float*>(bn + lo), 1);
    auto rd = [&](int i) __attribute__((always_inline)) { return i < NS ? rd_sd(bn, i) : rd_w(bc, i - NS); };
    u32x4 hp[2][2];  // fp16 copy of P for the slot (bf16 input)
    // P of query block qb, elements 4k .. 4k+3 (k = 0..3)
    auto p_chunk = [&](int qb, int k) __attribute__((always_inline)) {
      float p[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = fast_exp2(x[qb][4 * k + e] * scale_log2);
      const int i1 = k >> 1, q0 = 2 * (k & 1);
      pnxt[qb][i1][q0] = pack2<E>(p[0], p[1]);
      pnxt[qb][i1][q0 + 1] = pack2<E>(p[2], p[3]);
      if constexpr (!PF16) {
        hp[qb][i1][q0] = pack2<F16>(p[0], p[1]);
        hp[qb][i1][q0 + 1] = pack2<F16>(p[2], p[3]);
      }
      if (k & 1) *slot(t + 1, qb, i1) = PF16 ? pnxt[qb][i1] : hp[qb][i1];
    };
    constexpr int PD = 3;
    u32x4 rot[PD + 1];
#pragma unroll
    for (int i = 0; i < PD; ++i) rot[i] = rd(i);
    // S of block 0 is complete after MFMA NS - 2, of block 1 after NS - 1; P's four
    // chunks of a block go out every SP-th dV MFMA from C0 (block 0) and C1 (block 1)
    // (D = 128: 17, 19, 21, 23 and 25 .. 31)
    constexpr int SP = NV / 8, C0 = NS + SP - 1, C1 = C0 + NV / 2;
    static_for<0, NT>([&](auto I) __attribute__((always_inline)) {
      constexpr int i = decltype(I)::value;
      if constexpr (i + PD < NT) rot[(i + PD) % (PD + 1)] = rd(i + PD);
      if constexpr (i % 2 == 0 && i / 2 <= 2 * NDMA)
        if (dm) dma_part(job, i / 2);
      if constexpr (i < NS) {
        x[i & 1] = mfma32<E>(rot[i % (PD + 1)], xf[i >> 1], x[i & 1]);
      } else {
        constexpr int j = i - NS, qb = j / (2 * DB), db = (j >> 1) % DB, i1 = j & 1;
        acc[db] = mfma32<E>(rot[i % (PD + 1)], pcur[qb][i1], acc[db]);
      }
      if constexpr (i >= C0 && i < C0 + 4 * SP && (i - C0) % SP == 0) p_chunk(0, (i - C0) / SP);
      if constexpr (i >= C1 && i < C1 + 4 * SP && (i - C1) % SP == 0) p_chunk(1, (i - C1) / SP);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  auto stream1 = [&](int t) __attribute__((always_inline)) {  // (role 1 issues no DMA)
    const unsigned char* bn = bufp(t + 1);
    const unsigned char* bc = bufp(t);
    u32x4 w[2][2], bop[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) w[qb][i1] = *slot(t, qb, i1);
    auto rd = [&](int i) __attribute__((always_inline)) { return i < NV ? rd_w(bc, i) : rd_sd(bn, i - NV); };
    // dS of query block qb, elements 4k .. 4k+3
    auto ds_chunk = [&](int qb, int k) __attribute__((always_inline)) {
      const int i1 = k >> 1, q0 = 2 * (k & 1);
#pragma unroll
      for (int q = q0; q < q0 + 2; ++q) {
        const int g = 8 * i1 + 2 * q;
        const uint32_t v = w[qb][i1][q];
        bop[qb][i1][q] = pack2<E>(mul_f16_f32<0>(v, x[qb][g]), mul_f16_f32<1>(v, x[qb][g + 1]));
      }
    };
    constexpr int PD = 3;
    u32x4 rot[PD + 1];
#pragma unroll
    for (int i = 0; i < PD; ++i) rot[i] = rd(i);
    // block 1's dS under block 0's dK MFMAs when there are 8 of them (D = 128); with
    // fewer, all of dS first
    constexpr bool DS1_IN = NV >= 16;
#pragma unroll
    for (int k = 0; k < 4; ++k) ds_chunk(0, k);
    if constexpr (!DS1_IN)
#pragma unroll
      for (int k = 0; k < 4; ++k) ds_chunk(1, k);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NT>([&](auto I) __attribute__((always_inline)) {
      constexpr int i = decltype(I)::value;
      if constexpr (i + PD < NT) rot[(i + PD) % (PD + 1)] = rd(i + PD);
      if constexpr (DS1_IN && i < 4) ds_chunk(1, i);
      if constexpr (i == NV / 2) {  // dS is formed: x takes dP(t+1) - Delta
        x[0] = load_rows(reinterpret_cast<const float*>(bn + lo), 0);
        x[1] = load_rows(reinterpret_cast<const float*>(bn + lo), 1);
      }
      if constexpr (i < NV) {
        constexpr int qb = i / (2 * DB), db = (i >> 1) % DB, i1 = i & 1;
        acc[db] = mfma32<E>(rot[i % (PD + 1)], bop[qb][i1], acc[db]);
      } else {
        constexpr int j = i - NV;
        x[j & 1] = mfma32<E>(rot[i % (PD + 1)], xf[j >> 1], x[j & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // per item: the next item's descriptor, the edge-pair count, the prologue
  auto begin_item = [&](int k) __attribute__((always_inline)) {
    const int Ln = item_L(k + 1);
    has_next = Ln >= 0;
    if (has_next) {
      const KItem it = make_item(Ln, k + 1);
      n_u = it.u;
      n_jt = it.jt;
      n_bh0 = it.bh0;
      n_i0 = it.i0;
      n_hc = it.hc;
      n_rev = it.rev;
      n_tb = it.tb;
      n_te = it.te;
      n_base = it.base;
    }
    set_edges();
    prologue();
  };
  // to the next item: its first pair at position te is in flight if iteration te - 2
  // ran, its second at te + 1 if iteration te - 1 ran (which also loaded its K/V rows)
  auto next_item = [&]() __attribute__((always_inline)) {
    const int nn = n_te - n_tb;
    pre = ((te - tb >= 2 && nn >= 1) ? 1 : 0) | ((te - tb >= 1 && nn >= 2) ? 2 : 0);
    xf_pre = te - tb >= 1;
    boff = ((boff + te - n_tb) % NBUF + NBUF) % NBUF;
    first = false;
    set_item(KItem{n_u, n_jt, n_bh0, n_i0, n_hc, n_rev, n_tb, n_te, n_base});
  };

  // The two roles run separate loops with the same barriers per item, so each keeps
  // only its own state in registers.  Role 0 alternates the two packed-P register
  // sets by unrolling two pairs.
  if (role == 0) {
    auto step = [&](int t, u32x4 (&pc)[2][2], u32x4 (&pn)[2][2], auto full) __attribute__((always_inline)) {
      top(t);
      if (t + 1 < te) front(t + 1, x, pn, full);
      back(t, x, pc, full);
    };
    auto step_mv = [&](int t, auto full) __attribute__((always_inline)) {
      step(t, pk, pkn, full);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) pk[qb][i1] = pkn[qb][i1];
    };
    for (int k = 0;; ++k) {
      begin_item(k);
      // (E1f: the full pairs whose successor, if any, is full as well)
      const int E1f = E1 < te ? E1 - 1 : E1;
      int t = tb;
      for (; t < E0; ++t) step_mv(t, BTag<false>{});  // leading edge pairs
      for (; t + 2 < E1; t += 2) {
        sync();
        stream0(t, pk, pkn);
        sync();
        stream0(t + 1, pkn, pk);
      }
      for (; t < E1f; ++t) step_mv(t, BTag<true>{});
      for (; t < te; ++t) step_mv(t, BTag<false>{});  // trailing edge pairs
      epilogue();
      if (!has_next) break;
      next_item();
    }
  } else {
    auto step1 = [&](int t, auto full) __attribute__((always_inline)) {
      top(t);
      back(t, x, pk, full);
      if (t + 1 < te) front(t + 1, x, pkn, full);
    };
    for (int k = 0;; ++k) {
      begin_item(k);
      const int E1f = E1 < te ? E1 - 1 : E1;
      int t = tb;
      for (; t < E0; ++t) step1(t, BTag<false>{});
      for (; t + 1 < E1; ++t) {
        sync();
        stream1(t);
      }
      for (; t < E1f; ++t) step1(t, BTag<true>{});
      for (; t < te; ++t) step1(t, BTag<false>{});
      epilogue();
      if (!has_next) break;
      next_item();
    }
  }
}

// ===========================================================================
// dQ
// ===========================================================================
// Waves per SIMD the dQ kernel is register-budgeted for: two whenever two
// workgroups fit in LDS with every SIMD holding two waves (measured 25% faster
// at D = 128, tile 128 x 64, than one wave with a larger register budget).
template <int D, int BM, int BN>
constexpr int dq_waves_per_simd() {
  return (D <= 64 || (BM == 128 && BN == 64)) ? 2 : 1;
}

template <typename E, int D, int BM, int BN>
__global__ __launch_bounds__(2 * BM)
__attribute__((amdgpu_waves_per_eu(dq_waves_per_simd<D, BM, BN>(), dq_waves_per_simd<D, BM, BN>())))
void dq_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
               const uint16_t* __restrict__ V, const uint16_t* __restrict__ O,
               const uint16_t* __restrict__ dO, const float* __restrict__ Lse,
               uint16_t* __restrict__ dQ, float* __restrict__ Rb, int B, int H, int Hkv, int S,
               float scale_log2, float sm_scale) {
  constexpr int NW = BM / 32;
  constexpr int NB = BN / 32, KT = D / 16, DB = D / 32;
  constexpr int ROWB = D * 2, CPR = ROWB / 16;
  constexpr int TILE = BN * ROWB;
  constexpr int NBLK = TILE / 1024;
  static_assert(TILE % 1024 == 0, "tiles are whole 1 KB DMA blocks");
  const float NEG_INF = -__builtin_inff();

  __shared__ __attribute__((aligned(1024))) unsigned char lds0[2 * TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char lds1[2 * TILE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hh = lane >> 5;

  // work item: (b, h, query tile), XCD aware as the forward: XCD wg % 8 takes a
  // contiguous range of (b, h) and walks them in groups of xcd_group() heads, heaviest
  // query tiles of the group first (at B=4 H=32 S=4096 D=128, against all 16 heads of
  // the XCD at once: one (b, h) after another -1.4 %, groups of 4 +1.5 %, and about
  // 1 % over groups of 8)
  const int nq = (S + BM - 1) / BM;
  const int nunits = B * H;
  const int wg = blockIdx.x;
  int bh, qt;
  if (nunits % 8 == 0) {
    const int per = nunits / 8, i = wg / 8;
    const int G = xcd_group(per, nq);
    const int grp = i / (G * nq), r = i % (G * nq);
    bh = (wg % 8) * per + grp * G + r % G;
    qt = nq - 1 - r / G;
  } else {
    bh = wg % nunits;
    qt = nq - 1 - wg / nunits;
  }
  const size_t base = (size_t)bh * S * D;
  // query head h reads K/V head h / (H / Hkv)
  const size_t kvbase = (size_t)((bh / H) * Hkv + (bh % H) / (H / Hkv)) * S * D;
  const unsigned char* Kb = reinterpret_cast<const unsigned char*>(K + kvbase);
  const unsigned char* Vb = reinterpret_cast<const unsigned char*>(V + kvbase);

  const int r0 = qt * BM, q0 = r0 + 32 * wave, m = q0 + c;
  const int ntiles = min((r0 + BM + BN - 1) / BN, (S + BN - 1) / BN);  // keys >= S are never needed
  const int jfull = r0 / BN;


  // Q and dO rows as B operands; Delta = rowsum(dO * O) from the same row halves
  u32x4 qf[KT], dof[KT];
  float delta;
  {
    const size_t mr = (size_t)min(m, S - 1) * D;  // rows >= S: any valid row, never stored
    const uint16_t* qr = Q + base + mr + 8 * hh;
    const uint16_t* dr = dO + base + mr + 8 * hh;
    const uint16_t* orr = O + base + mr + 8 * hh;
    float part = 0.f;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      qf[t] = gload16(qr + 16 * t);
      dof[t] = gload16(dr + 16 * t);
      const u32x4 o = gload16(orr + 16 * t);
#pragma unroll
      for (int w = 0; w < 4; ++w) part = dot_pair<E>(dof[t][w], o[w], part);
    }
    delta = halfwave_sum(part);
  }
  const float lse = Lse[(size_t)bh * S + min(m, S - 1)];
  // the dK/dV kernel's per-row terms, when it runs after this one: -LSE/c, -Delta
  if (Rb != nullptr && hh == 0 && m < S) {
    const float inv_c = 1.0f / scale_log2;
    Rb[(size_t)bh * S + m] = -lse * inv_c;
    Rb[(size_t)B * H * S + (size_t)bh * S + m] = -delta;
  }

  TileOffsets<ROWB> to;
  to.init(lane);

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

  // DMA of the K and V tiles of key tile j (row-major, swizzled) into an LDS buffer;
  // per-lane source offsets are fixed (dvo), the tile offset j*TILE is a scalar.
  constexpr int NDMA = (NBLK + NW - 1) / NW;
  const int drow = lane / CPR, dch = lane % CPR;
  int dvo[NDMA];
#pragma unroll
  for (int x = 0; x < NDMA; ++x) {
    const int row = (wave + x * NW) * (1024 / ROWB) + drow;
    dvo[x] = row * ROWB + ((dch ^ bswz(row, CPR)) << 4);
  }

  auto dma_tile = [&](int j, unsigned char* buf) __attribute__((always_inline)) {
    const int rows_b = min(TILE, S * ROWB - j * TILE);  // rows of a partial last tile past S read zero
    const auto krs = make_rsrc(Kb + (size_t)j * TILE, rows_b);
    const auto vrs = make_rsrc(Vb + (size_t)j * TILE, rows_b);
#pragma unroll
    for (int x = 0; x < NDMA; ++x) {
      const int blk = wave + x * NW;
      if (NBLK % NW == 0 || blk < NBLK) {
        dma16(krs, buf + blk * 1024, dvo[x], 0);
        dma16(vrs, buf + TILE + blk * 1024, dvo[x], 0);
      }
    }
  };

  auto compute = [&](const unsigned char* Ks, int k0, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(mask_tag)::value;
    const unsigned char* Vs = Ks + TILE;
    int nvalid = NB;
    if constexpr (MASKED) {
      nvalid = (q0 + 32 - k0) / 32;
      nvalid = nvalid > NB ? NB : nvalid;
      if (nvalid <= 0) return;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (MASKED && nb >= nvalid) continue;
      // S^T = K Q^T, dP^T = V dO^T: lane (c = query, hh), register g -> key 32nb + acc_row(g)
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const int o = to.opnd[t] + 32 * nb * ROWB;
        s = mfma32<E>(lds_read16(Ks, o), qf[t], s);
        dp = mfma32<E>(lds_read16(Vs, o), dof[t], dp);
      }
      const bool diag = MASKED && (k0 + 32 * nb == q0);
      float ds[16];
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        float x = s[g];
        if (diag && acc_row(g, hh) > c) x = NEG_INF;
        const float p = fast_exp2(__builtin_fmaf(x, scale_log2, -lse));
        ds[g] = p * (dp[g] - delta);
      }
      u32x4 dsk[2];
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1)
#pragma unroll
        for (int q = 0; q < 4; ++q) dsk[i1][q] = pack2<E>(ds[8 * i1 + 2 * q], ds[8 * i1 + 2 * q + 1]);
      // dQ^T += K^T dS^T (k-slots: keys 32nb + 16i1 + 8r2 + 4hh + 0..3)
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) {
          const int u = 2 * nb + i1;
          acc[db] = mfma32<E>(tr_read2(Ks, to.tr(db, u, 0), to.tr(db, u, 1)), dsk[i1], acc[db]);
        }
    }
  };

  // Full tiles at D >= 64, pipelined by hand.  Left to itself the
  // compiler issues each MFMA's LDS operand read just before it and waits for it
  // (one read in flight).  Here a tile is a sequence of items, NB blocks of 32 keys
  // each made of KT/2 S/dP items (two k-steps: 2 S and 2 dP MFMAs) and DB/2 dQ
  // items (two d blocks x two key halves: 4 MFMAs), each item with 4 operands.
  // Item m's operands are read in the region of item m-2's MFMAs (three rotating
  // buffers, regions pinned by sched_barrier); P and dS of a block run in a region
  // of their own after its last S/dP item; a tile's last item runs at the start of
  // the next tile, under the operand reads that follow the barrier.  Same
  // arithmetic in the same order as compute() (bitwise equal).
  constexpr bool PIPE = (D >= 64);
  constexpr int IK = KT / 2, IB = IK + DB / 2, NITEM = NB * IB;
  u32x4 pb[3][4];
  u32x4 dsk_c[2];      // dS of the current block, kept for the deferred item
  f32x16 s_c, dp_c;
  auto rd_item = [&](const unsigned char* Ks, auto mt) __attribute__((always_inline)) {
    constexpr int m = decltype(mt)::value, nb = m / IB, k = m % IB, bi = m % 3;
    if constexpr (k < IK) {
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int o = to.opnd[2 * k + x] + 32 * nb * ROWB;
        pb[bi][2 * x] = lds_read16(Ks, o);
        pb[bi][2 * x + 1] = lds_read16(Ks + TILE, o);
      }
    } else {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) {
          const int db = 2 * (k - IK) + jj, u = 2 * nb + i1;
          pb[bi][2 * jj + i1] = tr_read2(Ks, to.tr(db, u, 0), to.tr(db, u, 1));
        }
    }
  };
  auto mm_item = [&](auto mt) __attribute__((always_inline)) {
    constexpr int m = decltype(mt)::value, k = m % IB, bi = m % 3;
    if constexpr (k < IK) {
      if constexpr (k == 0) {
        s_c = f32x16{};
        dp_c = f32x16{};
      }
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        s_c = mfma32<E>(pb[bi][2 * x], qf[2 * k + x], s_c);
        dp_c = mfma32<E>(pb[bi][2 * x + 1], dof[2 * k + x], dp_c);
      }
    } else {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i1 = 0; i1 < 2; ++i1) {
          const int db = 2 * (k - IK) + jj;
          acc[db] = mfma32<E>(pb[bi][2 * jj + i1], dsk_c[i1], acc[db]);
        }
    }
  };
  auto grad_block = [&]() __attribute__((always_inline)) {
    float ds[16];
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const float p = fast_exp2(__builtin_fmaf(s_c[g], scale_log2, -lse));
      ds[g] = p * (dp_c[g] - delta);
    }
#pragma unroll
    for (int i1 = 0; i1 < 2; ++i1)
#pragma unroll
      for (int q = 0; q < 4; ++q) dsk_c[i1][q] = pack2<E>(ds[8 * i1 + 2 * q], ds[8 * i1 + 2 * q + 1]);
  };
  auto tile_pipelined = [&](const unsigned char* Ks, auto prev) __attribute__((always_inline)) {
    rd_item(Ks, IC<0>{});
    rd_item(Ks, IC<1>{});
    if constexpr (decltype(prev)::value) mm_item(IC<NITEM - 1>{});   // the previous tile's last item
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NITEM - 1>([&](auto mt) __attribute__((always_inline)) {
      constexpr int m = decltype(mt)::value;
      if constexpr (m + 2 < NITEM) rd_item(Ks, IC<m + 2>{});
      mm_item(mt);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (m % IB == IK - 1) {   // the block's S and dP are complete
        grad_block();
        __builtin_amdgcn_sched_barrier(0);
      }
    });
  };

  auto step = [&](int j, auto par_tag, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool P = decltype(par_tag)::value;
    unsigned char* cur = P ? lds1 : lds0;
    unsigned char* nxt = P ? lds0 : lds1;
    if (j + 1 < ntiles) dma_tile(j + 1, nxt);
    compute(cur, j * BN, mask_tag);
    __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
    __syncthreads();
  };
  // (full tiles only: j < jfull <= ntiles - 1, so tile j + 1 always exists and its DMA
  // needs no branch)
  auto step_pipelined = [&](int j, auto par_tag, auto prev) __attribute__((always_inline)) {
    constexpr bool P = decltype(par_tag)::value;
    unsigned char* cur = P ? lds1 : lds0;
    unsigned char* nxt = P ? lds0 : lds1;
    dma_tile(j + 1, nxt);
    tile_pipelined(cur, prev);
    __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
    __syncthreads();
  };

  dma_tile(0, lds0);
  __builtin_amdgcn_s_waitcnt(kBwdWaitVmcnt0);
  __syncthreads();
  int j = 0;
  if constexpr (PIPE) {
    if (jfull > 0) {
      step_pipelined(0, BTag<false>{}, BTag<false>{});
      for (j = 1; j + 1 < jfull; j += 2) {
        step_pipelined(j, BTag<true>{}, BTag<true>{});
        step_pipelined(j + 1, BTag<false>{}, BTag<true>{});
      }
      if (j < jfull) {
        step_pipelined(j, BTag<true>{}, BTag<true>{});
        ++j;
      }
      mm_item(IC<NITEM - 1>{});   // the last full tile's last item
    }
  } else {
    for (; j + 1 < jfull; j += 2) {
      step(j, BTag<false>{}, BTag<false>{});
      step(j + 1, BTag<true>{}, BTag<false>{});
    }
    if (j < jfull) {
      step(j, BTag<false>{}, BTag<false>{});
      ++j;
    }
  }
  for (; j < ntiles; ++j) {
    if (j & 1) step(j, BTag<true>{}, BTag<true>{});
    else step(j, BTag<false>{}, BTag<true>{});
  }

  if (m >= S) return;
  uint16_t* dqr = dQ + base + (size_t)m * D;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i1 = 0; i1 < 2; ++i1)
      gstore16(dqr + db * 32 + 16 * i1 + 8 * hh, pack8<E>(acc[db], 8 * i1, sm_scale));
}

// ===========================================================================
// dK / dV from per-chunk partial sums
// ===========================================================================
// dK[bkv, n, :] = sum over c < nsplit of Pk[bkv * nsplit + c, n, :] (and dV from
// Pv), in chunk order, rounded once to the element type.  One thread per 8
// consecutive d values; grid-stride over all B * Hkv * S * D / 8 of them.
template <typename E, int D>
__global__ __launch_bounds__(256)
void dkdv_reduce_kernel(const float* __restrict__ Pk, const float* __restrict__ Pv,
                       uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, int BHkv, int S, int nsplit) {
  const size_t per_head = (size_t)S * (D / 8);
  const size_t total = (size_t)BHkv * per_head;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const size_t bkv = i / per_head, r = i - bkv * per_head;
    f32x16 acc = f32x16{};   // [0, 8) dK, [8, 16) dV
    for (int c = 0; c < nsplit; ++c) {
      const size_t off = ((bkv * nsplit + c) * per_head + r) * 8;
      const f32x4 k0 = gload_f32x4(Pk + off), k1 = gload_f32x4(Pk + off + 4);
      const f32x4 v0 = gload_f32x4(Pv + off), v1 = gload_f32x4(Pv + off + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] += k0[e];
        acc[4 + e] += k1[e];
        acc[8 + e] += v0[e];
        acc[12 + e] += v1[e];
      }
    }
    gstore16(dK + i * 8, pack8<E>(acc, 0, 1.0f));
    gstore16(dV + i * 8, pack8<E>(acc, 8, 1.0f));
  }
}

// ===========================================================================
// Per-row terms without dQ: -LSE/c and -Delta of every query row into Rb
// ===========================================================================
// What dq_kernel stores for dK/dV when it runs first, for the order that runs dK/dV
// first (fa_bwd, or fa_bwd_gqa without a workspace): the same two lanes per row
// (lane c, half hh of D), the same v_dot2c order over the half's 8-wide pieces and the
// same sum of the halves, so the terms, and every gradient formed from them, equal
// that path's bitwise.  HBM-bound: reads O and dO once (4 D bytes per row) and LSE,
// writes 8 bytes per row.  One wave = 32 rows.
template <typename E, int D>
__global__ __launch_bounds__(256)
void rowterms_kernel(const uint16_t* __restrict__ O, const uint16_t* __restrict__ dO,
                     const float* __restrict__ Lse, float* __restrict__ Rb, int BH, int S, float scale_log2) {
  constexpr int KT = D / 16;
  const int lane = threadIdx.x & 63, c = lane & 31, hh = lane >> 5;
  const long long rows = (long long)BH * S;
  const long long row = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 32 + c;
  const long long r = row < rows ? row : rows - 1;   // lanes past the end compute a valid row, store nothing
  const uint16_t* dr = dO + r * D + 8 * hh;
  const uint16_t* orr = O + r * D + 8 * hh;
  float part = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const u32x4 d = gload16(dr + 16 * t);
    const u32x4 o = gload16(orr + 16 * t);
#pragma unroll
    for (int w = 0; w < 4; ++w) part = dot_pair<E>(d[w], o[w], part);
  }
  const float delta = halfwave_sum(part);
  if (hh == 0 && row < rows) {
    const float inv_c = 1.0f / scale_log2;
    Rb[row] = -Lse[row] * inv_c;
    Rb[rows + row] = -delta;
  }
}

template <typename E, int D>
static bool launch_rowterms(const BwdArgs& a, float* rb) {
  const long long rows = (long long)a.B * a.H * a.S;
  const int grid = (int)((rows + 127) / 128);
  hipLaunchKernelGGL((rowterms_kernel<E, D>), dim3(grid), dim3(256), 0, (hipStream_t)a.stream,
                     (const uint16_t*)a.o, (const uint16_t*)a.d_o, a.lse, rb, a.B * a.H, a.S, a.scale_log2);
  return hipGetLastError() == hipSuccess;
}

// ---------------------------------------------------------------------------
template <typename E, int D, int BMQ, int BNK>
static bool launch_dkdv(const BwdArgs& a) {
  static_assert(BNK == kDkdvKeys, "host split heuristics assume this key tile");
  const int nsplit = a.nsplit > 1 ? a.nsplit : 1;
  const dim3 grid(a.B * a.Hkv * nsplit * ((a.S + BNK - 1) / BNK)), block(2 * BNK);
  bool paired = false;
  // (the paired kernel's streams are written for any D; at D = 64 it measured slower
  // than the one-wave kernel, which already holds two waves per SIMD there: backward
  // -6.0 % at B=2 H=16 S=4096 fp16, -3.5 % MQA B=1 H=32 S=4096, -12.6 % B=4 H=32 bf16)
  if constexpr (FA_DKDV_PAIR && D == 128) {
    if (a.rowb) {
      // one workgroup per CU walks the key tiles (the kernel reads the grid size) on the
      // alternating walk.  Against the upward walk (the kernel's earlier form) the
      // alternating one first paid where a K/V head's query heads of Q and dO fill the
      // 4 MiB L2 (D = 128 bf16 backward: B=2 H=32 S=4096 with G = 4 +3.9 %, B=1 H=32
      // S=4096 MQA +10.3 %, B=1 H=32 S=8192 G = 8 +7.6 %, MHA S=8192 B=2 H=32 / B=1 H=32 /
      // B=1 H=16 +3.2 / +3.6 / +1.8 %; MHA S=4096 B=4 H=32 -1.0 %); with its DMA issued by
      // the role-0 waves it pays at every size measured (MHA B=4 H=32 S=4096 +0.9 % in three
      // runs, B=2 / B=1 H=32 S=4096 +0.5 / +1.4 %, B=4 H=32 S=2048 / 1024 +0.2 / +2.2 %,
      // B=2 H=16 S=2048 +0.5 %, B=2 H=8 S=2048 +0.6 %, B=1 H=8 S=4096 +0.6 %)
      const auto kern = dkdv_pair_kernel<E, D, BMQ, BNK>;
      static const int per_cu = occupancy_per_cu((const void*)kern, 4 * BNK);
      const dim3 pgrid(resident_grid((int)grid.x, per_cu));
      hipLaunchKernelGGL(kern, pgrid, dim3(4 * BNK), 0, (hipStream_t)a.stream,
                         (const uint16_t*)a.q, (const uint16_t*)a.k, (const uint16_t*)a.v, (const uint16_t*)a.d_o,
                         a.rowb, (uint16_t*)a.dk, (uint16_t*)a.dv, a.wsk, a.wsv,
                         nsplit, a.B, a.H, a.Hkv, a.S, a.scale_log2, a.sm_scale);
      paired = true;
    }
  }
  if (!paired && a.rowb)
    hipLaunchKernelGGL((dkdv_kernel<E, D, BMQ, BNK, true>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.q, (const uint16_t*)a.k, (const uint16_t*)a.v, (const uint16_t*)a.o,
                       (const uint16_t*)a.d_o, a.lse, a.rowb, (uint16_t*)a.dk, (uint16_t*)a.dv, a.wsk, a.wsv,
                       nsplit, a.B, a.H, a.Hkv, a.S, a.scale_log2, a.sm_scale);
  else if (!paired)
    hipLaunchKernelGGL((dkdv_kernel<E, D, BMQ, BNK, false>), grid, block, 0, (hipStream_t)a.stream,
                       (const uint16_t*)a.q, (const uint16_t*)a.k, (const uint16_t*)a.v, (const uint16_t*)a.o,
                       (const uint16_t*)a.d_o, a.lse, nullptr, (uint16_t*)a.dk, (uint16_t*)a.dv, a.wsk, a.wsv,
                       nsplit, a.B, a.H, a.Hkv, a.S, a.scale_log2, a.sm_scale);
  if (hipGetLastError() != hipSuccess) return false;
  if (nsplit > 1) {
    const size_t threads = (size_t)a.B * a.Hkv * a.S * (D / 8);
    const int grid = (int)std::min<size_t>((threads + 255) / 256, 8192);
    hipLaunchKernelGGL((dkdv_reduce_kernel<E, D>), dim3(grid), dim3(256), 0, (hipStream_t)a.stream,
                       a.wsk, a.wsv, (uint16_t*)a.dk, (uint16_t*)a.dv, a.B * a.Hkv, a.S, nsplit);
    if (hipGetLastError() != hipSuccess) return false;
  }
  return true;
}

template <typename E, int D, int BM, int BN>
static bool launch_dq(const BwdArgs& a) {
  hipLaunchKernelGGL((dq_kernel<E, D, BM, BN>), dim3(a.B * a.H * ((a.S + BM - 1) / BM)), dim3(2 * BM), 0,
                     (hipStream_t)a.stream, (const uint16_t*)a.q, (const uint16_t*)a.k,
                     (const uint16_t*)a.v, (const uint16_t*)a.o, (const uint16_t*)a.d_o, a.lse,
                     (uint16_t*)a.dq, a.rowb, a.B, a.H, a.Hkv, a.S, a.scale_log2, a.sm_scale);
  return hipGetLastError() == hipSuccess;
}

// tile_m / tile_n set the dQ kernel's query rows per workgroup and keys per LDS
// tile.  The dK/dV kernel always runs 4 waves (128 keys) per workgroup over
// 64-row query tiles: with its K/V rows and two accumulators in registers it
// holds one wave per SIMD at D = 128, and this shape keeps every SIMD busy and
// the triple-buffered Q/dO/O tiles inside LDS for every head dim.
// With a row-terms buffer the dQ kernel runs first and leaves -LSE/c and -Delta
// of every query row there (it forms Delta once per row, from rows it holds in
// registers anyway); the dK/dV kernel then stages those instead of the O tiles.
// Without one, dK/dV runs first and forms Delta from O and dO in every workgroup.
template <typename E, int D, int BMQ, int BNK>
static int launch_bwd(const BwdArgs& a) {
  if (a.rowb) {
    if (!launch_dq<E, D, BMQ, BNK>(a)) return FA_ERR_LAUNCH;
    return launch_dkdv<E, D, 64, 128>(a) ? FA_OK : FA_ERR_LAUNCH;
  }
  // dK/dV first: dQ's own output buffer holds the per-row terms until dQ, which runs
  // last and forms its own, overwrites it (8 bytes per row in a 2 D-byte row).  With
  // form_delta (the study entry's variant) dK/dV forms them in every key tile instead.
  if (!a.form_delta && (reinterpret_cast<uintptr_t>(a.dq) & 15) == 0) {
    BwdArgs t = a;
    t.rowb = static_cast<float*>(a.dq);
    if (!launch_rowterms<E, D>(t, t.rowb) || !launch_dkdv<E, D, 64, 128>(t)) return FA_ERR_LAUNCH;
    return launch_dq<E, D, BMQ, BNK>(a) ? FA_OK : FA_ERR_LAUNCH;
  }
  if (!launch_dkdv<E, D, 64, 128>(a)) return FA_ERR_LAUNCH;
  return launch_dq<E, D, BMQ, BNK>(a) ? FA_OK : FA_ERR_LAUNCH;
}

template <typename E, int D>
static BwdFn pick_bwd(int bm, int bn) {
  if (bm == 64 && bn == 64) return launch_bwd<E, D, 64, 64>;
  if (bm == 64 && bn == 128) return launch_bwd<E, D, 64, 128>;
  if (bm == 128 && bn == 64) return launch_bwd<E, D, 128, 64>;
  if (bm == 128 && bn == 128) return launch_bwd<E, D, 128, 128>;
  return nullptr;
}

}  // namespace fa

// FA_ETYPE (fa::F16 / fa::BF16), FA_D and FA_BWD_TABLE come from the build.
extern "C" FA_HIDDEN fa::BwdFn FA_BWD_TABLE(int bm, int bn) {
  return fa::pick_bwd<FA_ETYPE, FA_D>(bm, bn);
}
