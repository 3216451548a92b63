// fa_device.h - gfx950 building blocks shared by the forward and backward kernels.
//
// Conventions used throughout (CDNA3/CDNA4 32x32 MFMA, wave64):
//   lane l = 32*hh + c, with c = l % 32 and hh = l / 32.
//   v_mfma_f32_32x32x16_{bf16,f16}: C[32x32] += A[32x16] * B[16x32]
//     A operand: lane holds row c,    8 consecutive k of k-half hh (16 bytes)
//     B operand: lane holds column c, 8 consecutive k of k-half hh (16 bytes)
//     C/D accumulator (16 fp32): register g of lane (c, hh) is
//       C[row = 8*(g/4) + 4*hh + (g%4)][col = c]
//   A and B use the same (hh, slot) -> k assignment, so any permutation of the
//   contraction index applied to both operands leaves the product unchanged.
//
// Row permutation pi: when the rows of an A operand are fed in the order
//   A row r <- logical row pi(r), pi swapping bits 2 and 3 of r,
// accumulator register g of lane (c, hh) holds logical row
//   16*(g/8) + 8*hh + (g%8),
// i.e. registers 0..7 cover 8 consecutive logical rows (8*hh .. 8*hh+7) and
// registers 8..15 the next 8 of the upper 16.  The kernels use this so that a
// score accumulator can be fed straight back as the next MFMA's operand, and
// so that an output accumulator stores 16 contiguous bytes per lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fa {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Element tags: storage is raw 16-bit words; the tag picks MFMA flavour and
// fp32 -> 16-bit rounding (round-to-nearest-even for both).
struct F16 {};
struct BF16 {};

__host__ __device__ __forceinline__ int pi_swap23(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

template <typename E>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c);

template <>
__device__ __forceinline__ f32x16 mfma32<BF16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x16 mfma32<F16>(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_{bf16,f16}: C[16x16] += A[16x32] * B[32x16]; lane l holds
// row / column l % 16 of A / B with k = 8 (l / 16) .. + 7, and C registers r of
// lane l hold row 4 (l / 16) + r, column l % 16.
template <typename E>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c);

template <>
__device__ __forceinline__ f32x4 mfma16<BF16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma16<F16>(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

// Two 16-bit ones in one word.
template <typename E>
constexpr uint32_t ones2() {
  return std::is_same<E, BF16>::value ? 0x3F803F80u : 0x3C003C00u;
}

// Two fp32 -> one 32-bit word holding two 16-bit values (x in the low half).
template <typename E>
__device__ __forceinline__ uint32_t pack2(float x, float y);

template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float x, float y) {
  bf16x2 v = {(__bf16)x, (__bf16)y};
  return __builtin_bit_cast(uint32_t, v);
}

template <>
__device__ __forceinline__ uint32_t pack2<F16>(float x, float y) {
  f16x2 v = {(_Float16)x, (_Float16)y};
  return __builtin_bit_cast(uint32_t, v);
}

// acc + (sum of the two 16-bit values packed in w): v_dot2c_f32_{bf16,f16}
// against the pair (1, 1), i.e. one instruction for two adds.
template <typename E>
__device__ __forceinline__ float add_pair(uint32_t w, float acc);

template <>
__device__ __forceinline__ float add_pair<BF16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3F803F80u),
                                         acc, false);
}

template <>
__device__ __forceinline__ float add_pair<F16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, 0x3C003C00u), acc, false);
}

// acc + a.lo * b.lo + a.hi * b.hi for two packed 16-bit pairs (v_dot2c_f32_*).
template <typename E>
__device__ __forceinline__ float dot_pair(uint32_t a, uint32_t b, float acc);

template <>
__device__ __forceinline__ float dot_pair<BF16>(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
}

template <>
__device__ __forceinline__ float dot_pair<F16>(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
}

// The fp16 value in half `hi` of w, times x, in fp32 (v_fma_mix_f32 with a -0
// addend: the widening is exact and the product rounds once, as in a widening
// conversion followed by v_mul_f32, in one instruction instead of two).
template <int HI>
__device__ __forceinline__ float mul_f16_f32(uint32_t w, float x) {
  // (the compiler folds fma(a, b, -0) into a multiply and keeps the widening apart)
  float r;
  const float nz = -0.0f;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(x), "v"(nz));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(x), "v"(nz));
  return r;
}

// One 16-bit element -> fp32.
template <typename E>
__device__ __forceinline__ float to_f32(uint32_t bits16);

template <>
__device__ __forceinline__ float to_f32<BF16>(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

template <>
__device__ __forceinline__ float to_f32<F16>(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// 8 accumulator registers [base, base+8) -> 16 bytes of packed 16-bit values.
template <typename E>
__device__ __forceinline__ u32x4 pack8(const f32x16& v, int base, float mul) {
  u32x4 r;
  r[0] = pack2<E>(v[base + 0] * mul, v[base + 1] * mul);
  r[1] = pack2<E>(v[base + 2] * mul, v[base + 3] * mul);
  r[2] = pack2<E>(v[base + 4] * mul, v[base + 5] * mul);
  r[3] = pack2<E>(v[base + 6] * mul, v[base + 7] * mul);
  return r;
}

// Value of the other half-wave (lane l ^ 32) combined with this lane's:
// v_permlane32_swap exchanges lanes 32..63 of one operand with lanes 0..31 of
// the other; feeding x twice yields {x_lo, x_hi} in every lane.
__device__ __forceinline__ float halfwave_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float halfwave_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum over the 4 lanes of a lane quad (DPP quad_perm [1,0,3,2] then [2,3,0,1]).
__device__ __forceinline__ float quad_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
  return x;
}

// Units (heads, or head groups) an XCD works on at one time when its workgroups walk
// `per` units of `nq` query tiles each: four, or the largest power of two below four
// that divides `per`.  Measured against groups of about 256 workgroups (8 units at
// B=4 H=32 S=4096, where nq = 32): forward +2.2 % and backward +1.1 % at B=4 H=32
// S=4096 D=128 bf16; GQA B=2 H=32 H_kv=8 S=8192 and MQA B=1 H=32 S=16384 D=64 equal;
// groups of two units lose 6.5 % on the forward at B=2 H=16 S=4096 D=64 fp16.
__device__ __forceinline__ int xcd_group(int per, int nq) {
  (void)nq;
  int g = 1;
  while (2 * g <= 4 && per % (2 * g) == 0) g *= 2;
  return g;
}

__device__ __forceinline__ u32x4 lds_read16(const unsigned char* base, int byte_off) {
  return *reinterpret_cast<const u32x4*>(base + byte_off);
}

__device__ __forceinline__ void lds_write16(unsigned char* base, int byte_off, const u32x4& v) {
  *reinterpret_cast<u32x4*>(base + byte_off) = v;
}

__device__ __forceinline__ void lds_write8(unsigned char* base, int byte_off, const u32x2& v) {
  *reinterpret_cast<u32x2*>(base + byte_off) = v;
}

// Buffer descriptor for raw byte-addressed loads from [p, p + bytes): word 3 =
// 0x00020000 is the gfx9 setting for untyped dword access; loads past `bytes`
// (vector offset) read zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// Global -> LDS DMA of 16 bytes per lane (buffer_load_dwordx4 ... lds): lane L
// reads rsrc bytes [voff + soff, +16) and writes them to lds + 16 L.
// (Kept out of kernel bodies: clang's host pass drops a kernel's launch stub
// when these builtins appear inside the kernel's own lambdas.)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, unsigned char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// The same DMA for 4 bytes per lane (buffer_load_dword ... lds): lane L's word
// lands at lds + 4 L.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rs, unsigned char* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 4, voff, soff, 0, 0);
}

__device__ __forceinline__ u32x4 gload16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ void gstore16(uint16_t* p, const u32x4& v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
__device__ __forceinline__ void gstore_f32x4(float* p, const f32x4& v) {
  *reinterpret_cast<f32x4*>(p) = v;
}
__device__ __forceinline__ f32x4 gload_f32x4(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}

// ---------------------------------------------------------------------------
// LDS tile layouts.
//
// Row-major tile  [R][C] of 16-bit values, rows of C*2 bytes split in 16-byte
// chunks.  Chunk ch of row r is stored at chunk position ch ^ rm_swz(r):
//   rm_swz(r) = pi_swap23(r) & 7 (masked to the chunk count).
// An MFMA operand read of 32 rows fed in pi order (lane c reads row
// base + pi(c)) then touches 8 distinct 16-byte bank groups per 8 lanes.
template <int C>
__device__ __forceinline__ int rm_off(int r, int ch) {
  constexpr int CH = C / 8;
  constexpr int MASK = (CH >= 8 ? 8 : CH) - 1;
  return r * (C * 2) + ((ch ^ (pi_swap23(r) & MASK)) << 4);
}

// Transposed tile: logical [R][C] stored as [C][R] (R contiguous), filled from
// row-major global memory 4 rows x 8 columns per thread item and read as MFMA
// operands with 8 consecutive R values per lane.  Chunk ch of stored row x is
// placed at ch ^ tr_swz(x), tr_swz(x) = (pi_swap23(x) & 7) ^ ((x >> 3) & 7);
// this keeps both the pi-ordered operand reads and the 8-byte transposing
// writes free of bank conflicts (16 lanes of a write hit 16 distinct slots).
template <int R>
__device__ __forceinline__ int tr_off(int x, int ch) {
  static_assert(R % 64 == 0, "transposed tile needs >= 8 chunks per stored row");
  return x * (R * 2) + ((ch ^ ((pi_swap23(x) & 7) ^ ((x >> 3) & 7))) << 4);
}

// Item i of a transposed fill covers global rows 4*g .. 4*g+3 and columns
// 8*cc .. 8*cc+7.  Within each group of 16 items: 4 column chunks x 4 row
// groups, so a 16-lane write phase is conflict free and the global loads of a
// wave cover whole 64-byte segments.
template <int C>
__device__ __forceinline__ void tr_item(int i, int& g, int& cc) {
  constexpr int CB = C / 32;  // column blocks of 4 chunks
  const int t16 = i & 15, blk = i >> 4;
  cc = (blk % CB) * 4 + (t16 & 3);
  g = (blk / CB) * 4 + (t16 >> 2);
}

// Write the 4x8 item (rows 4g..4g+3, columns 8cc..8cc+7, given as four
// 16-byte row pieces) transposed into a [C][R] tile.
template <int R>
__device__ __forceinline__ void tr_write(unsigned char* tile, int g, int cc, const u32x4 (&v)[4]) {
  const int ch = g >> 1, half = (g & 1) << 3;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int w = e >> 1;
    u32x2 out;
    if (e & 1) {
      out[0] = (v[0][w] >> 16) | (v[1][w] & 0xFFFF0000u);
      out[1] = (v[2][w] >> 16) | (v[3][w] & 0xFFFF0000u);
    } else {
      out[0] = (v[0][w] & 0xFFFFu) | (v[1][w] << 16);
      out[1] = (v[2][w] & 0xFFFFu) | (v[3][w] << 16);
    }
    const int x = cc * 8 + e;
    lds_write8(tile, tr_off<R>(x, ch) + half, out);
  }
}

}  // namespace fa
