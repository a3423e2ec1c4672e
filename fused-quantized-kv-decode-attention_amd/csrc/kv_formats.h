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

#include <type_traits>

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

// Raw buffer access (gfx9 descriptor word 3 = 0x00020000, stride 0):
// loads whose byte offset is at or past num_records return zeros.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int CPOL_SC1 = 16;  // cache-policy bit: device-scope coherent access
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
template <int BYTES>
__device__ __forceinline__ auto buf_load(rsrc_t r, uint32_t off) {
  if constexpr (BYTES == 16) {
    return __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
  } else if constexpr (BYTES == 8) {
    return __builtin_bit_cast(u2_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
  } else {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
  }
}

template <int FMT, int D>
struct Fmt;

// ---------------------------------------------------------------- fp16 ----
template <int D>
struct Fmt<KV_F16, D> {
  static constexpr bool QUANT = false;
  static constexpr int ROWB = 2 * D;  // bytes per token row
  static constexpr int NKI = D / 32;  // MFMA steps per tile
  using KT = u4_t;                    // one K load
  static constexpr int KL = D / 32;   // K loads per lane per tile
  // Step i, lane group kb reads row bytes [64 i + 16 kb, +16): each load
  // instruction covers 64 contiguous bytes of 16 rows.
  __host__ __device__ static constexpr uint32_t klane(int kb) { return 16 * kb; }
  __device__ static void load_k(rsrc_t r, uint32_t off, KT (&kr)[KL]) {
#pragma unroll
    for (int j = 0; j < KL; ++j) kr[j] = buf_load<16>(r, off + 64 * j);
  }
  __device__ static h8_t kfrag(const KT (&kr)[KL], int i) { return __builtin_bit_cast(h8_t, kr[i]); }
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return 32 * i + 8 * kb + e;
  }
  // Query operand for step i: the same eight head-dim elements as kfrag.
  __device__ static h8_t qfrag(rsrc_t rq, uint32_t row_elem, int i, int kb) {
    return __builtin_bit_cast(h8_t, buf_load<16>(rq, 2u * (row_elem + kd_index(i, kb, 0))));
  }
  static constexpr int VB = 16;              // bytes per lane per V load
  static constexpr int LPR = ROWB / VB;      // lanes per token row
  static constexpr int TPL = 64 / LPR;       // tokens per wave load
  static constexpr int VLD = 16 / TPL;       // V loads per tile
  static constexpr int EV = 8;               // elements per lane per V load
  static constexpr float VBIAS = 0.0f;
  __device__ static void vconv(const u4_t vd, float (&f)[EV]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // element copied to a scalar first: this compiler's __builtin_bit_cast of
      // a vector-element expression reads element 0 whatever the index
      const uint32_t x = vd[k];
      const h2_t h = __builtin_bit_cast(h2_t, x);
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
  using KT = u4_t;
  static constexpr int KL = D / 64;
  // Load j, lane group kb reads row bytes [64 j + 16 kb, +16) = two MFMA steps.
  __host__ __device__ static constexpr uint32_t klane(int kb) { return 16 * kb; }
  __device__ static void load_k(rsrc_t r, uint32_t off, KT (&kr)[KL]) {
#pragma unroll
    for (int j = 0; j < KL; ++j) kr[j] = buf_load<16>(r, off + 64 * j);
  }
  __device__ static h8_t kfrag(const KT (&kr)[KL], int i) {
    const u4_t v = kr[i / 2];
    h2_t a, b, c, d;
    i8x4_to_h2x2((i % 2) ? v.z : v.x, a, b);
    i8x4_to_h2x2((i % 2) ? v.w : v.y, c, d);
    return h8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  }
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return 64 * (i / 2) + 16 * kb + 8 * (i % 2) + e;
  }
  __device__ static h8_t qfrag(rsrc_t rq, uint32_t row_elem, int i, int kb) {
    return __builtin_bit_cast(h8_t, buf_load<16>(rq, 2u * (row_elem + kd_index(i, kb, 0))));
  }
  static constexpr int VB = 16;
  static constexpr int LPR = ROWB / VB;
  static constexpr int TPL = 64 / LPR;
  static constexpr int VLD = 16 / TPL;
  static constexpr int EV = 16;
  static constexpr float VBIAS = 128.0f;  // vconv yields x + 128
  __device__ static void vconv(const u4_t vd, float (&f)[EV]) {
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
  // one load of ROWB/4 bytes (one dword = 8 elements per MFMA step)
  using KT = typename std::conditional<D == 128, u4_t, u2_t>::type;
  static constexpr int KL = 1;
  // Lane group kb reads row bytes [ROWB/4 * kb, +ROWB/4): four lanes cover a row.
  __host__ __device__ static constexpr uint32_t klane(int kb) { return (ROWB / 4) * kb; }
  __device__ static void load_k(rsrc_t r, uint32_t off, KT (&kr)[KL]) {
    kr[0] = buf_load<sizeof(KT)>(r, off);
  }
  __device__ static h8_t kfrag(const KT (&kr)[KL], int i) {
    h2_t h[4];
    i4x8_to_h2x4(kr[0][i], h);
    return h8_t{h[0].x, h[0].y, h[1].x, h[1].y, h[2].x, h[2].y, h[3].x, h[3].y};
  }
  // slot e of step i holds element 8 i + {0,2,4,6,1,3,5,7}[e] of the lane's run
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return (D / 4) * kb + 8 * i + (e < 4 ? 2 * e : 2 * (e - 4) + 1);
  }
  __device__ static h8_t qfrag(rsrc_t rq, uint32_t row_elem, int i, int kb) {
    const h8_t v = __builtin_bit_cast(h8_t, buf_load<16>(rq, 2u * (row_elem + kd_index(i, kb, 0))));
    return h8_t{v[0], v[2], v[4], v[6], v[1], v[3], v[5], v[7]};
  }
  static constexpr int VB = (D == 128) ? 16 : 8;
  static constexpr int LPR = ROWB / VB;  // 4
  static constexpr int TPL = 64 / LPR;   // 16
  static constexpr int VLD = 16 / TPL;   // 1
  static constexpr int EV = 2 * VB;
  static constexpr float VBIAS = 8.0f;   // vconv yields n + 8
  template <typename VT>
  __device__ static void vconv(const VT vd, float (&f)[EV]) {
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

template <int VB>
using vraw_t = typename std::conditional<VB == 16, u4_t, u2_t>::type;

template <int FMT, int D>
__device__ __forceinline__ vraw_t<Fmt<FMT, D>::VB> load_v(rsrc_t r, uint32_t off) {
  return buf_load<Fmt<FMT, D>::VB>(r, off);
}

}  // namespace fqkv
