// KV-cache formats as seen by the gfx950 decode kernels.
//
// One 16-token tile of a KV row block is consumed two ways:
//   * K side: operand B of v_mfma_f32_16x16x32_f16. Lane l holds token
//     (l % 16) of the tile and 8 head-dim elements per MFMA step for lane
//     group kb = l / 16. Which head-dim element sits in which operand slot
//     is free (the contraction sums over all of them) as long as the query
//     fragment (operand A) uses the same map, kd_index(). Each format picks
//     the map that keeps its global loads wide and contiguous and its
//     int -> fp16 conversion cheap.
//   * V side: plain VALU. A token row is split over LPR lanes, each holding
//     VB contiguous bytes = EV elements; a wave covers TPL tokens per load.
//
// Exactness: int8 and int4 values become fp16 through the 0x6400 exponent
// trick (1024 + u is exact in fp16 for 0 <= u < 1024) followed by an exact
// subtraction, and become fp32 through v_cvt_f32_ubyte; both are exact, so
// the dequantised value (float)q * (float)scale
// (decode_attn_int8_mw.cu:24,31; decode_attn_int4.cu:21-23,29-31) is
// reproduced bit for bit by fqkv_dequant_kv, which calls these same helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fqkv {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

enum KvFormat : int { KV_F16 = 0, KV_I8 = 1, KV_I4 = 2 };

// Bytes {b_lo, b_hi} selected by `sel` from t, each placed under the fp16
// exponent byte 0x64: the half2 (1024 + b_lo, 1024 + b_hi).
// v_perm_b32 byte selector: 0-3 pick bytes of the second operand, 4-7 of the first.
__device__ __forceinline__ h2_t bytes_under_1024(uint32_t t, uint32_t sel) {
  return __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, t, sel));
}
constexpr uint32_t SEL_B01 = 0x04010400u;  // bytes 0,1 of t
constexpr uint32_t SEL_B23 = 0x04030402u;  // bytes 2,3 of t

// Four int8 in a dword -> two exact half2 (elements 0,1 and 2,3).
__device__ __forceinline__ void i8x4_to_h2x2(uint32_t w, h2_t& a, h2_t& b) {
  const uint32_t t = w ^ 0x80808080u;  // two's complement x -> x + 128 in [0, 255]
  const h2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
  a = bytes_under_1024(t, SEL_B01) - off;
  b = bytes_under_1024(t, SEL_B23) - off;
}

// Eight int4 (one dword, byte k = elements 2k (low nibble) and 2k+1) -> four
// exact half2 in the order [e0 e2 | e4 e6 | e1 e3 | e5 e7].
__device__ __forceinline__ void i4x8_to_h2x4(uint32_t w, h2_t (&h)[4]) {
  const uint32_t t = w ^ 0x88888888u;  // nibble n -> n + 8 (mod 16) in [0, 15]
  const uint32_t lo = t & 0x0F0F0F0Fu;
  const uint32_t hi = (t >> 4) & 0x0F0F0F0Fu;
  const h2_t off = {(_Float16)1032.0f, (_Float16)1032.0f};
  h[0] = bytes_under_1024(lo, SEL_B01) - off;
  h[1] = bytes_under_1024(lo, SEL_B23) - off;
  h[2] = bytes_under_1024(hi, SEL_B01) - off;
  h[3] = bytes_under_1024(hi, SEL_B23) - off;
}

__device__ __forceinline__ float ubyte_f(uint32_t w, int k) {
  return (float)((w >> (8 * k)) & 0xFFu);  // v_cvt_f32_ubyte{k}
}

template <int FMT, int D>
struct Fmt;

// ---------------------------------------------------------------- fp16 ----
template <int D>
struct Fmt<KV_F16, D> {
  static constexpr bool QUANT = false;
  static constexpr int ROWB = 2 * D;  // bytes per token row
  static constexpr int NKI = D / 32;  // MFMA steps per tile
  static constexpr int KDW = D / 8;   // K dwords per lane per tile
  // Step i, lane group kb reads row bytes [64 i + 16 kb, +16): each load
  // instruction covers 64 contiguous bytes of 16 rows.
  __device__ static void load_k(const uint8_t* row, int kb, uint32_t (&kd)[KDW]) {
#pragma unroll
    for (int j = 0; j < NKI; ++j) {
      const u4_t v = *reinterpret_cast<const u4_t*>(row + 64 * j + 16 * kb);
      kd[4 * j + 0] = v.x; kd[4 * j + 1] = v.y; kd[4 * j + 2] = v.z; kd[4 * j + 3] = v.w;
    }
  }
  __device__ static h8_t kfrag(const uint32_t (&kd)[KDW], int i) {
    u4_t v = {kd[4 * i], kd[4 * i + 1], kd[4 * i + 2], kd[4 * i + 3]};
    return __builtin_bit_cast(h8_t, v);
  }
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return 32 * i + 8 * kb + e;
  }
  static constexpr int VB = 16;              // bytes per lane per V load
  static constexpr int LPR = ROWB / VB;      // lanes per token row
  static constexpr int TPL = 64 / LPR;       // tokens per wave load
  static constexpr int VLD = 16 / TPL;       // V loads per tile
  static constexpr int EV = 8;               // elements per lane per V load
  static constexpr float VBIAS = 0.0f;
  __device__ static void vconv(const uint32_t (&vd)[VB / 4], float (&f)[EV]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const h2_t h = __builtin_bit_cast(h2_t, vd[k]);
      f[2 * k] = (float)h.x;
      f[2 * k + 1] = (float)h.y;
    }
  }
  __host__ __device__ static constexpr int vd_index(int lir, int e) { return EV * lir + e; }
};

// ---------------------------------------------------------------- int8 ----
template <int D>
struct Fmt<KV_I8, D> {
  static constexpr bool QUANT = true;
  static constexpr int ROWB = D;
  static constexpr int NKI = D / 32;
  static constexpr int KDW = D / 16;
  // Load j, lane group kb reads row bytes [64 j + 16 kb, +16) = two MFMA steps.
  __device__ static void load_k(const uint8_t* row, int kb, uint32_t (&kd)[KDW]) {
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
      const u4_t v = *reinterpret_cast<const u4_t*>(row + 64 * j + 16 * kb);
      kd[4 * j + 0] = v.x; kd[4 * j + 1] = v.y; kd[4 * j + 2] = v.z; kd[4 * j + 3] = v.w;
    }
  }
  __device__ static h8_t kfrag(const uint32_t (&kd)[KDW], int i) {
    h2_t a, b, c, d;
    i8x4_to_h2x2(kd[2 * i], a, b);
    i8x4_to_h2x2(kd[2 * i + 1], c, d);
    return h8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  }
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return 64 * (i / 2) + 16 * kb + 8 * (i % 2) + e;
  }
  static constexpr int VB = 16;
  static constexpr int LPR = ROWB / VB;
  static constexpr int TPL = 64 / LPR;
  static constexpr int VLD = 16 / TPL;
  static constexpr int EV = 16;
  static constexpr float VBIAS = 128.0f;  // vconv yields x + 128
  __device__ static void vconv(const uint32_t (&vd)[VB / 4], float (&f)[EV]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t t = vd[k] ^ 0x80808080u;
#pragma unroll
      for (int b = 0; b < 4; ++b) f[4 * k + b] = ubyte_f(t, b);
    }
  }
  __host__ __device__ static constexpr int vd_index(int lir, int e) { return EV * lir + e; }
};

// ---------------------------------------------------------------- int4 ----
template <int D>
struct Fmt<KV_I4, D> {
  static constexpr bool QUANT = true;
  static constexpr int ROWB = D / 2;
  static constexpr int NKI = D / 32;
  static constexpr int KDW = D / 32;  // one dword (8 elements) per MFMA step
  // Lane group kb reads row bytes [ROWB/4 * kb, +ROWB/4): four lanes cover a row.
  __device__ static void load_k(const uint8_t* row, int kb, uint32_t (&kd)[KDW]) {
    if constexpr (D == 128) {
      const u4_t v = *reinterpret_cast<const u4_t*>(row + 16 * kb);
      kd[0] = v.x; kd[1] = v.y; kd[2] = v.z; kd[3] = v.w;
    } else {
      const u2_t v = *reinterpret_cast<const u2_t*>(row + 8 * kb);
      kd[0] = v.x; kd[1] = v.y;
    }
  }
  __device__ static h8_t kfrag(const uint32_t (&kd)[KDW], int i) {
    h2_t h[4];
    i4x8_to_h2x4(kd[i], h);
    return h8_t{h[0].x, h[0].y, h[1].x, h[1].y, h[2].x, h[2].y, h[3].x, h[3].y};
  }
  // slot e of step i holds element 8 i + {0,2,4,6,1,3,5,7}[e] of the lane's run
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return (D / 4) * kb + 8 * i + (e < 4 ? 2 * e : 2 * (e - 4) + 1);
  }
  static constexpr int VB = (D == 128) ? 16 : 8;
  static constexpr int LPR = ROWB / VB;  // 4
  static constexpr int TPL = 64 / LPR;   // 16
  static constexpr int VLD = 16 / TPL;   // 1
  static constexpr int EV = 2 * VB;
  static constexpr float VBIAS = 8.0f;   // vconv yields n + 8
  __device__ static void vconv(const uint32_t (&vd)[VB / 4], float (&f)[EV]) {
#pragma unroll
    for (int k = 0; k < VB / 4; ++k) {
      const uint32_t t = vd[k] ^ 0x88888888u;
      const uint32_t lo = t & 0x0F0F0F0Fu;
      const uint32_t hi = (t >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        f[8 * k + 2 * b] = ubyte_f(lo, b);
        f[8 * k + 2 * b + 1] = ubyte_f(hi, b);
      }
    }
  }
  __host__ __device__ static constexpr int vd_index(int lir, int e) { return EV * lir + e; }
};

template <int FMT, int D>
__device__ __forceinline__ void load_v(const uint8_t* row, int lir, uint32_t (&vd)[Fmt<FMT, D>::VB / 4]) {
  using F = Fmt<FMT, D>;
  if constexpr (F::VB == 16) {
    const u4_t v = *reinterpret_cast<const u4_t*>(row + 16 * lir);
    vd[0] = v.x; vd[1] = v.y; vd[2] = v.z; vd[3] = v.w;
  } else {
    const u2_t v = *reinterpret_cast<const u2_t*>(row + 8 * lir);
    vd[0] = v.x; vd[1] = v.y;
  }
}

}  // namespace fqkv
