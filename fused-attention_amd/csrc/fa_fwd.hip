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
// average of the V rows it weights; and the reference point m is lazy: a tile's
// p is computed against the current m, and only if some row's sum of p over
// the tile exceeds 2^FA_RESCALE_THRESHOLD (or is not finite) is the tile's row
// max taken, acc and l rescaled and p recomputed.  Every p therefore stays
// <= 2^T, no row max is reduced on the common path, and O = acc / l and
// LSE = m + log2(l) do not depend on the reference point; because l sums the
// same rounded weights as acc, a row dominated by one key still reproduces
// that key's V row exactly.
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
//   * causal skipping: key tiles past the workgroup's last row are never loaded;
//     the tiles that meet the workgroup's diagonal run the full-tile schedule with
//     the mask applied arithmetically, and a wave whose rows lie wholly before the
//     last tile skips it.  The first reference point is S(0)'s row max, so no
//     tile starts on the rescale path.
//   * heavy-first, XCD-aware order: the 8 XCDs each take a contiguous range of
//     (batch, head-group) units and dispatch the heaviest (last) query tiles of
//     all their units first.
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
// p is recomputed against a fresh row max only when a row's sum of p over a
// tile exceeds 2^FA_RESCALE_THRESHOLD
#ifndef FA_RESCALE_THRESHOLD
#define FA_RESCALE_THRESHOLD 8
#endif
constexpr float kSumLimit = float(1 << FA_RESCALE_THRESHOLD);

template <int D, int BM, int BN, int GH>
constexpr int fwd_waves_per_simd() {
  return (BN == 64 && (BM / 32) * GH >= 4) ? 2 : 1;
}

// Compile-time marker of a pipeline iteration that runs wholly below the diagonal.
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

  // K buffers at [0, 2 TILE), V buffers at [2 TILE, 4 TILE)
  __shared__ __attribute__((aligned(1024))) unsigned char lds[4 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hh = lane >> 5;
  const int wh = wave % GH, wr = wave / GH;

  // ---- work item: (batch, head group, query tile).  Workgroups reach the 8 XCDs
  // round-robin (wg % 8); XCD x takes a contiguous range of units (its own L2 keeps
  // their K/V) and walks them in groups of xcd_group() units, each group query tile
  // major with the heaviest tiles first, so the light tiles fill the end of every
  // group and of the kernel, and the units whose K/V the XCD streams at one time stay
  // few.  At B=4 H=32 S=4096 D=128 (16 units per XCD), against one unit after another:
  // groups of 4 units about +6 %, groups of 8 about +4 %.
  const int nq = (S + BM - 1) / BM;  // the last query tile may be partial
  const int units_per_b = H / GH;
  const int nunits = B * units_per_b;
  const int wg = blockIdx.x;
  int unit, qt;
  if (nunits % 8 == 0) {
    const int per = nunits / 8, i = wg / 8;
    const int G = xcd_group(per, nq);
    const int grp = i / (G * nq), r = i % (G * nq);
    unit = (wg % 8) * per + grp * G + r % G;
    qt = nq - 1 - r / G;
  } else {
    unit = wg % nunits;
    qt = nq - 1 - wg / nunits;
  }
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
  // key tiles up to the workgroup's last row; keys >= S are never needed (each lies past
  // every valid query, so the causal mask already excludes it)
  const int ntiles = min((r0 + BM + BN - 1) / BN, (S + BN - 1) / BN);
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
  // one buffer descriptor per tile, sized to the rows below S: rows of a partial last
  // tile past S read as zero (the scalar offset is not range-checked, the size is)
  auto tile_rsrc = [&](const unsigned char* bh, int j) __attribute__((always_inline)) {
    return make_rsrc(bh + (size_t)j * TILE, min(TILE, S * ROWB - j * TILE));
  };
  auto dma_k = [&](int j, unsigned char* buf) __attribute__((always_inline)) {
    const auto rs = tile_rsrc(Kbh, j);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int blk = wave + i * NW;
      if (NBLK % NW == 0 || blk < NBLK) dma16(rs, buf + blk * 1024, kvo[i], 0);
    }
  };
  auto dma_v = [&](int j, unsigned char* buf) __attribute__((always_inline)) {
    const auto rs = tile_rsrc(Vbh, j);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int blk = wave + i * NW;
      if (NBLK % NW == 0 || blk < NBLK) dma16(rs, buf + blk * 1024, vvo[i], 0);
    }
  };

  // ---- Q^T operand in registers: k-step t holds Q[m][16t + 8hh .. +7]
  u32x4 qf[KT];
  {
    const uint16_t* qrow = Q + qbase + (size_t)min(m, S - 1) * D + 8 * hh;  // rows >= S: any valid row
#pragma unroll
    for (int t = 0; t < KT; ++t) qf[t] = gload16(qrow + 16 * t);
  }

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
  float mrun = NEG_INF;
  // Row sums of P on the matrix pipe.  Fed as the B operand of a 16x16x32 MFMA, a
  // k-step u of P^T puts query n's 16 keys (both half-waves) in the k groups 0 and
  // 2 of column n and query n + 16's in groups 1 and 3 (n = lane % 16); against the
  // 0/1 selector rsel (ones in lanes 0 and 32, row 0, and 17 and 49, row 1) the
  // product's row 0 / row 1 hold those two queries' sums: lane n, registers 0 and 1.
  // lsum keeps l in that layout.  One such MFMA per k-step replaces eight
  // v_dot2c_f32_*, each of which stalls the matrix pipe of its SIMD for about 16
  // cycles on gfx950 (an issue-rate probe), where the MFMA takes its 16.
  const uint32_t one = (lane == 0 || lane == 32 || lane == 17 || lane == 49) ? ones2<E>() : 0u;
  const u32x4 rsel = {one, one, one, one};
  f32x4 lsum = f32x4{};

  // ---- pipeline stages.  Every tile is computed whole (all NB 32-key blocks);
  // on the tiles that meet the workgroup's diagonal the keys past each row are
  // set to -inf arithmetically (mask_tile), so those tiles run the same
  // branch-free schedule as the tiles below the diagonal, at the price of the
  // MFMAs of blocks that lie wholly past a wave's rows.  With per-wave code for
  // each block count the diagonal-region tiles took about twice a full tile.

  // S^T = K Q^T: A row c <- key 32nb + c; register g of lane (c, hh) holds
  // key offset 8*(g/4) + 4*hh + (g%4) of the block, query c.
  auto s_tile = [&](const unsigned char* Ks, f32x16 (&s)[NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      f32x16 x = f32x16{};
#pragma unroll
      for (int t = 0; t < KT; ++t) x = mfma32<E>(lds_read16(Ks, koff[t] + nb * 32 * ROWB), qf[t], x);
      s[nb] = x;
    }
  };

  // Causal mask of the tile starting at key k0: key k0 + 32nb + 8(g/4) + 4hh + (g%4)
  // lies past row q0 + c exactly when 8(g/4) + (g%4) + (4hh - c) > q0 - k0 - 32nb.
  const int lane_kq = 4 * hh - c;
  auto mask_tile = [&](f32x16 (&s)[NB], int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int t = q0 - k0 - 32 * nb;
#pragma unroll
      for (int g = 0; g < 16; ++g)
        if (lane_kq > t - (8 * (g >> 2) + (g & 3))) s[nb][g] = NEG_INF;
    }
  };

  // Row max of a tile in scaled log2 units.
  auto tile_max = [&](const f32x16 (&s)[NB]) __attribute__((always_inline)) {
    float mx = NEG_INF;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int g = 0; g < 16; ++g) mx = fmaxf(mx, s[nb][g]);
    return halfwave_max(mx) * scale_log2;
  };

  // Move the reference point to mx (or keep it if larger): rescale acc and l.
  auto rescale_to = [&](float mx) __attribute__((always_inline)) {
    const float mnew = fmaxf(mrun, mx);
    const float alpha = fast_exp2(mrun - mnew);
    mrun = mnew;
    lsum[0] *= alpha;                    // query lane % 16: this lane's own alpha
    lsum[1] *= __shfl_xor(alpha, 16);    // query lane % 16 + 16
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g = 0; g < 16; ++g) acc[db][g] *= alpha;
  };

  // P^T as the B operand of the PV MFMAs: k-step u = 2nb + i1 holds
  // keys 32nb + 16i1 + 4hh + {0..3} (slots 0-3) and +8 (slots 4-7);
  // returns the tile's sums of the rounded P in lsum's layout.
  auto exp_tile = [&](const f32x16 (&s)[NB], u32x4 (&pk)[2 * NB]) __attribute__((always_inline)) {
    f32x4 ts = f32x4{};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float p[16];
#pragma unroll
      for (int g = 0; g < 16; ++g) p[g] = fast_exp2(__builtin_fmaf(s[nb][g], scale_log2, -mrun));
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) {
        u32x4 w;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          w[q] = pack2<E>(p[8 * i1 + 2 * q], p[8 * i1 + 2 * q + 1]);
        }
        pk[2 * nb + i1] = w;
        ts = mfma16<E>(rsel, w, ts);
      }
    }
    return ts;
  };

  // P of a tile against the lazy reference point, and the l update.  The
  // reference point starts at the first tile's row max (taken after S(0)), so
  // the first tile needs no rescale.
  auto softmax = [&](const f32x16 (&s)[NB], u32x4 (&pk)[2 * NB]) __attribute__((always_inline)) {
    f32x4 ts = exp_tile(s, pk);
    if (__builtin_amdgcn_ballot_w64(!(ts[0] <= kSumLimit && ts[1] <= kSumLimit))) {
      rescale_to(tile_max(s));
      ts = exp_tile(s, pk);
    }
    lsum[0] += ts[0];
    lsum[1] += ts[1];
  };

  // O^T += V^T P^T with the V^T operands read two MFMAs ahead (three rotating
  // buffers, pinned by sched_barrier), the first two before the softmax, and the
  // four d blocks' accumulators taking turns; operand rows are d = 32db + pi(row),
  // keys per slot as above.  Left to itself the compiler read one operand ahead
  // and waited on it before every MFMA (2 % slower).
  constexpr int NPV = DB * 2 * NB;
  u32x4 pvb[3];
  auto pv_read = [&](const unsigned char* Vs, int i) __attribute__((always_inline)) {
    const int db = i % DB, u = i / DB;
    const int o = ((db & 1) ? voff_odd : voff_even) + 64 * db + 16 * u * ROWB;
    return lds_read_tr16x2(Vs, o, o + 8 * ROWB);
  };
  auto pv_pre = [&](const unsigned char* Vs) __attribute__((always_inline)) {
    pvb[0] = pv_read(Vs, 0);
    pvb[1] = pv_read(Vs, 1);
  };
  auto pv_full = [&](const unsigned char* Vs, const u32x4 (&pk)[2 * NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
      if (i + 2 < NPV) pvb[(i + 2) % 3] = pv_read(Vs, i + 2);
      acc[i % DB] = mfma32<E>(pvb[i % 3], pk[i / DB], acc[i % DB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto Kbuf = [&](int j) __attribute__((always_inline)) { return lds + (j & 1) * TILE; };
  auto Vbuf = [&](int j) __attribute__((always_inline)) { return lds + 2 * TILE + (j & 1) * TILE; };

  // ---- software pipeline over key tiles.  Iteration j: wait for K(j+1) and
  // V(j), start the DMA of K(j+2) and V(j+1), then S(j+1) on the MFMA pipe
  // while the VALU turns S(j) into P(j), then PV(j).  K runs one tile ahead of
  // V; both are double-buffered.  (The body is one scope with restrict-qualified
  // buffers: the tiles read are never the DMA targets, so the compiler need not
  // wait for the DMA before the transposed reads.)
  // Iterations below the diagonal (ST) run only while tile j + 2 is below the
  // workgroup's first row (j + 2 < jfull <= ntiles - 1, and j + 3 <= jfull for the
  // second iteration of a pair): nothing is masked and the DMAs need no test
  // (without the branches the DMA issue joins the tile's schedule: 2.3 % faster at
  // B=4 H=32 S=4096 D=128).  The others (j + 1 < ntiles) mask S(j+1).
  auto body = [&](int j, const unsigned char* __restrict__ kcur, unsigned char* __restrict__ kdst,
                  const unsigned char* __restrict__ vcur, unsigned char* __restrict__ vdst,
                  f32x16 (&sc)[NB], f32x16 (&sn)[NB], auto st) __attribute__((always_inline)) {
    if constexpr (decltype(st)::value) {
      dma_k(j + 2, kdst);
    } else {
      if (j + 2 < ntiles) dma_k(j + 2, kdst);
    }
    dma_v(j + 1, vdst);
    u32x4 pk[2 * NB];
    s_tile(kcur, sn);
    if constexpr (!decltype(st)::value) mask_tile(sn, (j + 1) * BN);
    pv_pre(vcur);
    softmax(sc, pk);
    pv_full(vcur, pk);
  };
  auto iteration = [&](int j, f32x16 (&sc)[NB], f32x16 (&sn)[NB], auto st) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    body(j, Kbuf(j + 1), Kbuf(j), Vbuf(j), Vbuf(j + 1), sc, sn, st);
  };

  // prologue: K(0), V(0), K(1) in flight; S(0) and its row max, the first reference
  // point (key 0 lies at or below every row, so the max is finite)
  dma_k(0, Kbuf(0));
  dma_v(0, Vbuf(0));
  if (ntiles > 1) dma_k(1, Kbuf(1));
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  f32x16 sa[NB], sb[NB];
  s_tile(Kbuf(0), sa);
  if (jfull == 0) mask_tile(sa, 0);
  mrun = tile_max(sa);

  // tiles j with j + 1 < jfull: both S(j) and S(j+1) below the diagonal
  int j = 0;
  for (; j + 2 < jfull; j += 2) {
    iteration(j, sa, sb, Tag<true>{});
    iteration(j + 1, sb, sa, Tag<true>{});
  }
  // the diagonal region (at most BM / BN + 2 tiles): S(j+1) masked, then moved into place
  for (; j + 1 < ntiles; ++j) {
    iteration(j, sa, sb, Tag<false>{});
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) sa[nb] = sb[nb];
  }
  // the last tile (no S to start); a wave whose rows lie wholly before it skips it
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (q0 + 31 >= j * BN) {
    u32x4 pk[2 * NB];
    pv_pre(Vbuf(j));
    softmax(sa, pk);
    pv_full(Vbuf(j), pk);
  }

  // ---- epilogue: O = acc / l; lane holds d = 32db + 16i1 + 8hh + 0..7
  // l of query c from lane c % 16 (register 0 for c < 16, 1 above)
  const float l_lo = __shfl(lsum[0], c & 15), l_hi = __shfl(lsum[1], c & 15);
  const float ltot = c < 16 ? l_lo : l_hi;
  const float inv = 1.0f / ltot;
  uint16_t* orow = O + qbase + (size_t)m * D;
  if (m < S) {  // rows of a partial last query tile past S are not stored
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int i1 = 0; i1 < 2; ++i1) gstore16(orow + db * 32 + 16 * i1 + 8 * hh, pack8<E>(acc[db], 8 * i1, inv));
    }
    if (LSE && hh == 0) Lse[(size_t)(b * H + hq) * S + m] = mrun + __log2f(ltot);
  }
}

// ---------------------------------------------------------------------------
template <typename E, int D, int BM, int BN, int GH, bool LSE>
static int launch_fwd(const FwdArgs& a) {
  constexpr int NT = 64 * (BM / 32) * GH;
  const int total = a.B * (a.H / GH) * ((a.S + BM - 1) / BM);
  hipLaunchKernelGGL((fwd_kernel<E, D, BM, BN, GH, LSE>), dim3(total), dim3(NT), 0, (hipStream_t)a.stream,
                     (const uint16_t*)a.q, (const uint16_t*)a.k, (const uint16_t*)a.v,
                     (uint16_t*)a.o, a.lse, a.B, a.H, a.Hkv, a.S, a.scale_log2);
  return hipGetLastError() == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

// A slice builds as one object (FA_FWD_PART 0) or, where its instances want different
// machine schedulers, as two: part 1 the one-head instances and the slice's table, part 2
// the instances of two and four heads per workgroup, whose table part 1 calls for GQA.
// The D = 128 slices split so (the Makefile): the one-head kernel runs 0.9-2.2 % faster under
// the compiler's max-ILP scheduling strategy (B=4 H=32 S=4096 bf16, B=2 H=8 S=8192 fp16),
// the grouped ones 0.5-1.7 % slower (GQA B=2 H=32 H_kv=8 S=4096 / 8192, B=1 H=32 H_kv=4
// S=8192); at D <= 64 every instance runs slower under it (-1.8 to -4.6 %), so those slices
// stay whole under the default strategy.  Outputs are bitwise equal either way.
#ifndef FA_FWD_PART
#define FA_FWD_PART 0
#endif

// Dispatch over the compile-time parameters of one (element type, D) slice.
template <typename E, int D>
static FwdFn pick_fwd(int bm, int bn, int gh, bool lse) {
#define FA_CASE(BM_, BN_, GH_)                                                          \
  if (bm == BM_ && bn == BN_ && gh == GH_)                                             \
    return lse ? launch_fwd<E, D, BM_, BN_, GH_, true> : launch_fwd<E, D, BM_, BN_, GH_, false>;
#if FA_FWD_PART != 2
  FA_CASE(64, 64, 1) FA_CASE(64, 128, 1) FA_CASE(128, 64, 1) FA_CASE(128, 128, 1)
#endif
#if FA_FWD_PART != 1
  FA_CASE(64, 64, 2) FA_CASE(64, 128, 2) FA_CASE(128, 64, 2)
  FA_CASE(64, 64, 4)
#endif
#undef FA_CASE
  return nullptr;
}

}  // namespace fa

// FA_ETYPE (fa::F16 / fa::BF16), FA_D and FA_FWD_TABLE come from the build; part 1 also
// takes FA_FWD_TABLE_GROUPED, the table part 2 was built under.
#if FA_FWD_PART == 1
extern "C" FA_HIDDEN fa::FwdFn FA_FWD_TABLE_GROUPED(int bm, int bn, int gh, int lse);
extern "C" FA_HIDDEN fa::FwdFn FA_FWD_TABLE(int bm, int bn, int gh, int lse) {
  return gh == 1 ? fa::pick_fwd<FA_ETYPE, FA_D>(bm, bn, gh, lse != 0) : FA_FWD_TABLE_GROUPED(bm, bn, gh, lse);
}
#else
extern "C" FA_HIDDEN fa::FwdFn FA_FWD_TABLE(int bm, int bn, int gh, int lse) {
  return fa::pick_fwd<FA_ETYPE, FA_D>(bm, bn, gh, lse != 0);
}
#endif
