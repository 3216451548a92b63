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
//     l = l*alpha + rowsum(p)       (unrounded p)
//     acc = acc*alpha + p(rounded to the input type) . v
//   O = acc / l; optional LSE = m + log2(l) (fused_backward.py:169).
//
// MI355X mapping:
//   * one workgroup = GH query heads (sharing one K/V head) x BM query rows;
//     one wave = one head x 32 query rows; WR = BM/32 waves per head.
//   * each wave computes S^T = K Q^T (keys x queries) so a lane owns ONE query
//     row: row max / row sum are register-local plus one permlane32 swap, and the
//     accumulator is fed straight back as the B operand of O^T += V^T P^T.
//   * Q stays in registers for the whole loop; K (row-major) and V^T
//     (transposed on the LDS write) tiles are double-buffered in LDS; the next
//     tile's global loads are in flight while the current tile is computed.
//   * causal skipping at two levels: key tiles past the workgroup's last row are
//     never loaded, and each wave skips 32-key blocks past its own last row.
//   * heavy-first, XCD-aware order: the 8 XCDs each take a contiguous range of
//     (batch, head-group) units; inside a unit the last (heaviest) query tile
//     is dispatched first.
#include "fa_device.h"
#include "fa_launch.h"

namespace fa {

// Two waves per SIMD where the working set fits 256 VGPRs without spilling
// (64-key tiles with >= 4 waves per workgroup), otherwise one.
template <int D, int BM, int BN, int GH>
constexpr int fwd_waves_per_simd() {
  return (BN == 64 && (BM / 32) * GH >= 4) ? 2 : 1;
}

template <typename E, int D, int BM, int BN, int GH, bool LSE>
__global__ __launch_bounds__(64 * (BM / 32) * GH)
__attribute__((amdgpu_waves_per_eu(fwd_waves_per_simd<D, BM, BN, GH>(), fwd_waves_per_simd<D, BM, BN, GH>())))
void fwd_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ Lse,
    int B, int H, int Hkv, int S, float scale_log2) {
  constexpr int WR = BM / 32;
  constexpr int NT = 64 * WR * GH;
  constexpr int KCH = D / 8;                      // 16-byte chunks per K row
  constexpr int NB = BN / 32;                     // 32-key blocks per tile
  constexpr int KT = D / 16;                      // MFMA k-steps over D
  constexpr int DB = D / 32;                      // 32-row blocks of O^T
  constexpr int K_BYTES = BN * D * 2;
  constexpr int V_BYTES = D * BN * 2;
  constexpr int BUF_BYTES = K_BYTES + V_BYTES;
  constexpr int K_ITEMS = BN * KCH;               // 16-byte chunks per K tile
  constexpr int V_ITEMS = (BN / 4) * (D / 8);     // 4x8 items per V tile
  constexpr int K_PER = (K_ITEMS + NT - 1) / NT;
  constexpr int V_PER = (V_ITEMS + NT - 1) / NT;
  const float NEG_INF = -__builtin_inff();

  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
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

  const uint16_t* Kbh = K + (size_t)(b * Hkv + hkv) * S * D;
  const uint16_t* Vbh = V + (size_t)(b * Hkv + hkv) * S * D;
  const size_t qbase = (size_t)(b * H + hq) * S * D;

  const int r0 = qt * BM;          // first query row of this workgroup
  const int q0 = r0 + wr * 32;     // first query row of this wave
  const int m = q0 + c;            // this lane's query row

  // ---- Q^T operand in registers: k-step t holds Q[m][16t + 8hh .. +7]
  u32x4 qf[KT];
  {
    const uint16_t* qrow = Q + qbase + (size_t)m * D + 8 * hh;
#pragma unroll
    for (int t = 0; t < KT; ++t) qf[t] = gload16(qrow + 16 * t);
  }

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
  float mrun = NEG_INF, lrun = 0.f;

  const int ntiles = (r0 + BM + BN - 1) / BN;

  // ---- global -> register prefetch of one K/V tile
  u32x4 kpre[K_PER];
  u32x4 vpre[V_PER][4];
  auto load_tile = [&](int j) {
    const uint16_t* Kt = Kbh + (size_t)j * BN * D;
    const uint16_t* Vt = Vbh + (size_t)j * BN * D;
#pragma unroll
    for (int it = 0; it < K_PER; ++it) {
      const int i = tid + it * NT;
      if (K_ITEMS % NT == 0 || i < K_ITEMS) kpre[it] = gload16(Kt + (size_t)i * 8);
    }
#pragma unroll
    for (int it = 0; it < V_PER; ++it) {
      const int i = tid + it * NT;
      if (V_ITEMS % NT == 0 || i < V_ITEMS) {
        int g, cc;
        tr_item<D>(i, g, cc);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          vpre[it][rr] = gload16(Vt + (size_t)(4 * g + rr) * D + 8 * cc);
      }
    }
  };
  auto store_tile = [&](int buf) {
    unsigned char* Ks = smem + buf * BUF_BYTES;
    unsigned char* Vs = Ks + K_BYTES;
#pragma unroll
    for (int it = 0; it < K_PER; ++it) {
      const int i = tid + it * NT;
      if (K_ITEMS % NT == 0 || i < K_ITEMS) lds_write16(Ks, rm_off<D>(i / KCH, i % KCH), kpre[it]);
    }
#pragma unroll
    for (int it = 0; it < V_PER; ++it) {
      const int i = tid + it * NT;
      if (V_ITEMS % NT == 0 || i < V_ITEMS) {
        int g, cc;
        tr_item<D>(i, g, cc);
        tr_write<BN>(Vs, g, cc, vpre[it]);
      }
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int j = 0; j < ntiles; ++j) {
    const int buf = j & 1;
    const bool more = (j + 1 < ntiles);
    if (more) load_tile(j + 1);

    const int k0 = j * BN;
    // 32-key blocks of this tile whose first key is <= the wave's last row
    int nvalid = (q0 + 32 - k0) / 32;
    nvalid = nvalid < 0 ? 0 : (nvalid > NB ? NB : nvalid);

    if (nvalid > 0) {
      const unsigned char* Ks = smem + buf * BUF_BYTES;
      const unsigned char* Vs = Ks + K_BYTES;

      // S^T = K Q^T, 32 keys per block; A row c <- key 32*nb + pi(c)
      f32x16 s[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        s[nb] = f32x16{};
        if (nb < nvalid) {
          const int key = nb * 32 + pi_swap23(c);
#pragma unroll
          for (int t = 0; t < KT; ++t) {
            const u32x4 a = lds_read16(Ks, rm_off<D>(key, 2 * t + hh));
            s[nb] = mfma32<E>(a, qf[t], s[nb]);
          }
        }
      }

      // causal mask on the diagonal block: register g holds key offset
      // 16*(g/8) + 8*hh + (g%8) inside the block, the lane holds query c
      float mx = NEG_INF;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (nb < nvalid) {
          if (k0 + 32 * nb == q0) {
#pragma unroll
            for (int g = 0; g < 16; ++g) {
              const int koff = 16 * (g >> 3) + 8 * hh + (g & 7);
              if (koff > c) s[nb][g] = NEG_INF;
            }
          }
#pragma unroll
          for (int g = 0; g < 16; ++g) mx = fmaxf(mx, s[nb][g]);
        }
      }
      mx = halfwave_max(mx);
      const float mnew = fmaxf(mrun, mx * scale_log2);
      const float alpha = fast_exp2(mrun - mnew);

      // P^T packed as the B operand of the PV MFMAs: k-step u = 2*nb + i1
      // holds keys 32nb + 16i1 + 8hh + 0..7
      u32x4 pk[2 * NB];
      float lsum = 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (nb < nvalid) {
          float p[16];
#pragma unroll
          for (int g = 0; g < 16; ++g) {
            p[g] = fast_exp2(__builtin_fmaf(s[nb][g], scale_log2, -mnew));
            lsum += p[g];
          }
#pragma unroll
          for (int i1 = 0; i1 < 2; ++i1) {
            u32x4 w;
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = pack2<E>(p[8 * i1 + 2 * q], p[8 * i1 + 2 * q + 1]);
            pk[2 * nb + i1] = w;
          }
        }
      }
      lrun = lrun * alpha + lsum;
      mrun = mnew;

      // O^T += V^T P^T; A row c <- d = 32*db + pi(c)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int g = 0; g < 16; ++g) acc[db][g] *= alpha;
        const int d = db * 32 + pi_swap23(c);
#pragma unroll
        for (int u = 0; u < 2 * NB; ++u) {
          if ((u >> 1) < nvalid) {
            const u32x4 a = lds_read16(Vs, tr_off<BN>(d, 2 * u + hh));
            acc[db] = mfma32<E>(a, pk[u], acc[db]);
          }
        }
      }
    }

    if (more) {
      store_tile(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: O = acc / l, 16 contiguous bytes per lane per (db, i1)
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
  constexpr int SMEM = 2 * (BN * D * 2 + D * BN * 2);
  auto kern = fwd_kernel<E, D, BM, BN, GH, LSE>;
  if (!set_smem_once(reinterpret_cast<const void*>(kern), SMEM)) return FA_ERR_LAUNCH;
  const int total = a.B * (a.H / GH) * (a.S / BM);
  hipLaunchKernelGGL(kern, dim3(total), dim3(NT), SMEM, (hipStream_t)a.stream,
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
