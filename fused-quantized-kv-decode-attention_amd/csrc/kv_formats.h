// KV-cache formats as seen by the gfx950 decode kernels.
//
// A wave consumes a 16-token tile of a KV row block with two matrix-core
// products, scores first and then P.V, both with the token index where the
// hardware wants it without any data shuffling through LDS:
//   * K side: operand A of v_mfma_f32_16x16x32_f16 (scores transposed,
//     S^T = K Q^T). Lane l holds token (l % 16) of the tile and 8 head-dim
//     elements per MFMA step for lane group kb = l / 16. Which head-dim
//     element sits in which operand slot is free (the contraction sums over
//     all of them) as long as the query fragment (operand B) uses the same
//     map, kd_index(). Each format picks the map that keeps its global loads
//     wide and its int -> fp16 conversion cheap.
//   * V side: operand A of the P.V product (O^T += V^T P^T; the kernel puts
//     two tiles in one v_mfma_f32_16x16x32_f16, four operand slots each).
//     Lane (R = l / 16, i = l % 16) loads VBYTES = ROWB / 16 contiguous bytes
//     at byte VBYTES * i of tile row 4 j + R (j = 0..3: four loads per tile,
//     each covering 4 whole rows). A 4 x 4 exchange of those chunks between
//     lane rows and loads (v_permlane32_swap, v_permlane16_swap) leaves lane
//     (R, i) with tokens 4 R .. 4 R + 3 of head-dim elements VE * i .. + VE-1,
//     and element c of the four chunks is the lane's operand of PV step c
//     (VE = D / 16 steps per tile).
//
// Exactness: an int8 value x or int4 value n enters the matrix cores as the
// fp16 subnormal (x + 128) * 2^-24 or (n + 8) * 2^-24 (an int4 high nibble,
// masked in place, as 16 (n + 8) * 2^-24): the biased integer sits in the
// mantissa under a zero exponent field, one byte permute or one three-input
// bitwise op per two values and no floating-point instruction. The matrix
// cores take fp16 subnormal operands as they are (products are exact in
// fp32), so a score comes out as 2^-24 (q.k + B sum(q)) and an output
// element as 2^-24 (w.v + B sum(w)) with the format's bias B; the kernel
// subtracts B sum(q) per score and B sum(w) once at the end. The operand
// times unit() is the biased integer exactly, which is how fqkv_dequant_kv,
// calling these same helpers, reproduces the reference's dequantised value
// (float)q * (float)scale (decode_attn_int8_mw.cu:24,31;
// decode_attn_int4.cu:21-23,29-31) bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fqkv {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

enum KvFormat : int { KV_F16 = 0, KV_I8 = 1, KV_I4 = 2, KV_BF16 = 3, KV_FP8 = 4 };

// v_perm_b32 byte selector: 0-3 pick bytes of the second operand, 4-7 of
// the first, 0x0C gives a zero byte.
constexpr uint32_t SEL_B01 = 0x0C010C00u;  // bytes 0, 1 of the second operand, each under a zero byte
constexpr uint32_t SEL_B23 = 0x0C030C02u;  // bytes 2, 3 likewise

// Four int8 in a dword -> two half2 of subnormals (x + 128) * 2^-24
// (elements 0,1 and 2,3): two's complement x ^ 0x80 = x + 128 in [0, 255],
// each byte placed under a zero high byte.
__device__ __forceinline__ void i8x4_to_h2x2(uint32_t w, h2_t& a, h2_t& b) {
  const uint32_t t = w ^ 0x80808080u;
  a = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0u, t, SEL_B01));
  b = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0u, t, SEL_B23));
}

// Two int4 of a dword -> half2 of subnormals, one bitwise op each: the
// nibbles at bits 0-3 and 16-19 (nib_lo) or 4-7 and 20-23 (nib_hi) are
// masked out with the sign bit flipped (n ^ 8 = n + 8 in [0, 15]), giving
// (n + 8) * 2^-24 or 16 (n + 8) * 2^-24.
__device__ __forceinline__ h2_t nib_lo(uint32_t t) {
  return __builtin_bit_cast(h2_t, (t & 0x000F000Fu) ^ 0x00080008u);
}
__device__ __forceinline__ h2_t nib_hi(uint32_t t) {
  return __builtin_bit_cast(h2_t, (t & 0x00F000F0u) ^ 0x00800080u);
}

// Eight int4 (one dword, byte k = elements 2k (low nibble) and 2k+1) -> four
// half2 in the order [e0 e4 | e1 e5 | e2 e6 | e3 e7]: even elements at 2^-24
// per unit, odd ones at 2^-20.
__device__ __forceinline__ void i4x8_to_h2x4(uint32_t w, h2_t (&h)[4]) {
  const uint32_t w2 = w >> 8;
  h[0] = nib_lo(w);
  h[1] = nib_hi(w);
  h[2] = nib_lo(w2);
  h[3] = nib_hi(w2);
}

// Raw buffer access (gfx9 descriptor word 3 = 0x00020000, stride 0):
// loads whose byte offset is at or past num_records return zeros.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int CPOL_SC0 = 1;   // cache-policy bit: bypass the CU's L1 (coherent within one XCD's L2)
constexpr int CPOL_SC1 = 16;  // cache-policy bit: device-scope coherent access
constexpr int CPOL_NT = 2;    // cache-policy bit: non-temporal (streaming) access
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// off goes in the VGPR offset, soff (wave-uniform) in the SGPR offset; the
// range check covers both (and the immediate field).
template <int BYTES>
__device__ __forceinline__ auto buf_load(rsrc_t r, uint32_t off, uint32_t soff = 0) {
  if constexpr (BYTES == 16) {
    return __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, 0));
  } else if constexpr (BYTES == 8) {
    return __builtin_bit_cast(u2_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, (int)soff, 0));
  } else if constexpr (BYTES == 4) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, (int)soff, 0);
  } else {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, (int)soff, 0);
  }
}

// V chunk of VBYTES bytes as VD dwords (a 2-byte chunk is zero-extended).
// V rows are read whole by one instruction stream and never again: the loads
// carry the non-temporal hint (CP = CPOL_NT) unless the caller asks for none
// (CP = 0).
template <int VBYTES, int VD, int CP = CPOL_NT>
__device__ __forceinline__ void load_vchunk(rsrc_t r, uint32_t off, uint32_t (&d)[VD], uint32_t soff = 0) {
  if constexpr (VBYTES == 16) {
    const u4_t v =
        __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, CP));
#pragma unroll
    for (int k = 0; k < 4; ++k) d[k] = v[k];
  } else if constexpr (VBYTES == 8) {
    const u2_t v = __builtin_bit_cast(u2_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, (int)soff, CP));
    d[0] = v[0];
    d[1] = v[1];
  } else if constexpr (VBYTES == 4) {
    d[0] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, (int)soff, CP);
  } else {
    d[0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, (int)soff, CP);
  }
}

// Common V-side geometry (ROWB bytes per token row, D head-dim elements).
template <int ROWB_, int D_>
struct VGeom {
  static constexpr int VBYTES = ROWB_ / 16;                 // bytes per lane per load
  static constexpr int VD = VBYTES >= 4 ? VBYTES / 4 : 1;   // dwords per lane per load
  static constexpr int VE = D_ / 16;                        // elements per chunk = PV steps
  static constexpr int EPD = (D_ / 16 + VD - 1) / VD;        // elements per dword
};

template <int FMT, int D>
struct Fmt;

// ---------------------------------------------------------------- fp16 ----
// fp16 K is staged through LDS: a tile's rows are loaded whole (lane group
// of ROWB / 16 lanes per row, 1 KiB of contiguous rows per instruction, with
// the streaming hint) and read back from LDS in the operand-A layout below.
// Loaded directly in that layout, each instruction touches 64 bytes of 16
// rows, which streamed ~6 % slower than whole rows on MI355X at batch 1.
template <int D>
struct Fmt<KV_F16, D> {
  static constexpr bool QUANT = false;   // per-token scales
  static constexpr bool BIASED = false;  // operands carry x + BIAS in units (integer codes)
  static constexpr bool BF16 = false;  // operands are fp16 bit patterns
  static constexpr bool STAGE_K = true;
  // tile offsets in the loads' SGPR offset (instead of VGPR adds per load):
  // for the VALU-bound int4 only; the scalar work ahead of the first loads
  // measured 3-5 % slower for fp16 and no faster for int8
  static constexpr bool SOFF_TILE = false;
  static constexpr int ROWB = 2 * D;  // bytes per token row
  static constexpr int NKI = D / 32;  // MFMA steps per tile
  using KT = u4_t;                    // one K load
  static constexpr int KL = D / 32;   // K loads per lane per tile
  static constexpr int LPR = ROWB / 16;   // lanes per row in a whole-row load
  static constexpr int RPL = 64 / LPR;    // rows per whole-row load (KL * RPL = 16)
  static constexpr int KPITCH = ROWB + 16;  // LDS row pitch: the padding spreads rows over the banks
  static constexpr int KSTAGE = 16 * KPITCH;  // LDS bytes per wave
  // Lane l's byte offset within a tile for the whole-row loads: row l / LPR
  // (plus RPL per load), bytes 16 (l % LPR).
  __device__ static uint32_t krow_lane(int lane, uint32_t ts) {
    return (uint32_t)(lane / LPR) * ts + 16u * (uint32_t)(lane % LPR);
  }
  __device__ static void load_k_rows(rsrc_t r, uint32_t off, uint32_t ts, KT (&kr)[KL], uint32_t soff = 0) {
#pragma unroll
    for (int j = 0; j < KL; ++j)
      kr[j] = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off + (uint32_t)(j * RPL) * ts), (int)soff, CPOL_NT));
  }
  // Through the wave's LDS rows: the whole-row registers in, the operand-A
  // registers (lane (kb, n): row n, bytes 16 kb + 64 j) out.
  __device__ static void stage_k(uint8_t* lds, int lane, KT (&kr)[KL]) {
#pragma unroll
    for (int j = 0; j < KL; ++j)
      *reinterpret_cast<u4_t*>(lds + (j * RPL + lane / LPR) * KPITCH + 16 * (lane % LPR)) = kr[j];
#pragma unroll
    for (int j = 0; j < KL; ++j)
      kr[j] = *reinterpret_cast<const u4_t*>(lds + (lane & 15) * KPITCH + 16 * (lane >> 4) + 64 * j);
  }
  // Step i, lane group kb reads row bytes [64 i + 16 kb, +16): each load
  // instruction covers 64 contiguous bytes of 16 rows.
  __host__ __device__ static constexpr uint32_t klane(int kb) { return 16 * kb; }
  __device__ static void load_k(rsrc_t r, uint32_t off, KT (&kr)[KL], uint32_t soff = 0) {
#pragma unroll
    for (int j = 0; j < KL; ++j) kr[j] = buf_load<16>(r, off + 64 * j, soff);
  }
  __device__ static h8_t kfrag(const KT (&kr)[KL], int i) { return __builtin_bit_cast(h8_t, kr[i]); }
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return 32 * i + 8 * kb + e;
  }
  // Query operand for step i: the same eight head-dim elements as kfrag.
  __device__ static h8_t qfrag(rsrc_t rq, uint32_t row_elem, int i, int kb) {
    return __builtin_bit_cast(h8_t, buf_load<16>(rq, 2u * (row_elem + kd_index(i, kb, 0))));
  }
  __device__ static uint32_t vprep(uint32_t x) { return x; }
  // element pos (0, 1) of dwords a and b -> half2 (a_pos, b_pos)
  __device__ static h2_t vpair(uint32_t a, uint32_t b, int pos) {
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(b, a, pos ? 0x07060302u : 0x05040100u));
  }
};

// ---------------------------------------------------------------- bf16 ----
// bf16 K and V move exactly like fp16 (16-bit elements: the same loads, LDS
// staging and exchanges, the same bit patterns in the operand registers); only
// the matrix-core products differ, which take bf16 operands: the query as a
// bf16 pair hi + lo (exact) and the weights as one (to 2^-16 relative).
template <int D>
struct Fmt<KV_BF16, D> : Fmt<KV_F16, D> {
  static constexpr bool BF16 = true;
};

// ---------------------------------------------------------------- int8 ----
template <int D>
struct Fmt<KV_I8, D> {
  static constexpr bool QUANT = true;
  static constexpr bool BIASED = true;
  static constexpr bool BF16 = false;
  static constexpr bool STAGE_K = false;
  static constexpr bool SOFF_TILE = false;
  static constexpr int ROWB = D;
  static constexpr int NKI = D / 32;
  using KT = u4_t;
  static constexpr int KL = D / 64;
  // operand value * unit = x + BIAS (every K slot and V element)
  static constexpr float BIAS = 128.0f;
  __host__ __device__ static constexpr float kunit(int) { return 16777216.0f; }
  __host__ __device__ static constexpr float vunit(int) { return 16777216.0f; }
  // Load j, lane group kb reads row bytes [64 j + 16 kb, +16) = two MFMA steps.
  __host__ __device__ static constexpr uint32_t klane(int kb) { return 16 * kb; }
  __device__ static void load_k(rsrc_t r, uint32_t off, KT (&kr)[KL], uint32_t soff = 0) {
#pragma unroll
    for (int j = 0; j < KL; ++j) kr[j] = buf_load<16>(r, off + 64 * j, soff);
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
  // a V dword before vpair: x ^ 0x80 = x + 128 in every byte
  __device__ static uint32_t vprep(uint32_t x) { return x ^ 0x80808080u; }
  // byte pos of prepared dwords a and b -> half2 of subnormals (a_pos, b_pos):
  // each byte placed under a zero high byte
  __device__ static h2_t vpair(uint32_t a, uint32_t b, int pos) {
    const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + pos) << 16) | (uint32_t)pos;
    return __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(b, a, sel));
  }
};

// ----------------------------------------------------------------- fp8 ----
// OCP fp8 e4m3 codes (1 byte per element, as int8) with fp16 per-token
// scales. gfx950 converts two codes to an fp16 pair in one instruction
// (v_cvt_scalef32_pk_f16_fp8, scale 1), exactly: every e4m3 value is an fp16
// value. So the operands are the true code values, with no bias and unit 1;
// everything else (loads, scale handling, the weight shift) is int8's.
__device__ __forceinline__ h2_t fp8x2_lo(uint32_t w) {
  return __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}
__device__ __forceinline__ h2_t fp8x2_hi(uint32_t w) {
  return __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
}

template <int D>
struct Fmt<KV_FP8, D> : Fmt<KV_I8, D> {
  static constexpr bool BIASED = false;
  static constexpr float BIAS = 0.0f;
  __host__ __device__ static constexpr float kunit(int) { return 1.0f; }
  __host__ __device__ static constexpr float vunit(int) { return 1.0f; }
  __device__ static h8_t kfrag(const u4_t (&kr)[D / 64], int i) {
    const u4_t v = kr[i / 2];
    const uint32_t x = (i % 2) ? v.z : v.x, y = (i % 2) ? v.w : v.y;
    const h2_t a = fp8x2_lo(x), b = fp8x2_hi(x), c = fp8x2_lo(y), d = fp8x2_hi(y);
    return h8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  }
  __device__ static uint32_t vprep(uint32_t x) { return x; }
  // byte pos of dwords a and b -> half2 (a_pos, b_pos): the two codes into
  // bytes 0 and 1, then one conversion
  __device__ static h2_t vpair(uint32_t a, uint32_t b, int pos) {
    const uint32_t sel = 0x0C0C0000u | ((uint32_t)(4 + pos) << 8) | (uint32_t)pos;
    return fp8x2_lo(__builtin_amdgcn_perm(b, a, sel));
  }
};

// ---------------------------------------------------------------- int4 ----
template <int D>
struct Fmt<KV_I4, D> {
  static constexpr bool QUANT = true;
  static constexpr bool BIASED = true;
  static constexpr bool BF16 = false;
  static constexpr bool STAGE_K = false;
  static constexpr bool SOFF_TILE = true;
  static constexpr int ROWB = D / 2;
  static constexpr int NKI = D / 32;
  // one load of ROWB/4 bytes (one dword = 8 elements per MFMA step)
  using KT = typename std::conditional<D == 128, u4_t, u2_t>::type;
  static constexpr int KL = 1;
  // operand value * unit = n + BIAS: K slots 2, 3, 6, 7 of a step and odd V
  // elements of a dword (high nibbles) sit 16 times higher
  static constexpr float BIAS = 8.0f;
  __host__ __device__ static constexpr float kunit(int e) { return ((e >> 1) & 1) ? 1048576.0f : 16777216.0f; }
  __host__ __device__ static constexpr float vunit(int pos) { return (pos & 1) ? 1048576.0f : 16777216.0f; }
  // Lane group kb reads row bytes [ROWB/4 * kb, +ROWB/4): four lanes cover a row.
  __host__ __device__ static constexpr uint32_t klane(int kb) { return (ROWB / 4) * kb; }
  __device__ static void load_k(rsrc_t r, uint32_t off, KT (&kr)[KL], uint32_t soff = 0) {
    kr[0] = buf_load<sizeof(KT)>(r, off, soff);
  }
  __device__ static h8_t kfrag(const KT (&kr)[KL], int i) {
    h2_t h[4];
    i4x8_to_h2x4(kr[0][i], h);
    return h8_t{h[0].x, h[0].y, h[1].x, h[1].y, h[2].x, h[2].y, h[3].x, h[3].y};
  }
  // slot e of step i holds element 8 i + {0,4,1,5,2,6,3,7}[e] of the lane's run
  __host__ __device__ static constexpr int kd_index(int i, int kb, int e) {
    return (D / 4) * kb + 8 * i + e / 2 + 4 * (e % 2);
  }
  // the query elements facing high nibbles are divided by 16 (exact unless
  // the quotient is an fp16 subnormal), so every product carries 2^-24
  __device__ static h8_t qfrag(rsrc_t rq, uint32_t row_elem, int i, int kb) {
    const h8_t v = __builtin_bit_cast(h8_t, buf_load<16>(rq, 2u * (row_elem + kd_index(i, kb, 0))));
    auto q16 = [](_Float16 x) { return (_Float16)((float)x * 0.0625f); };
    return h8_t{v[0], v[4], q16(v[1]), q16(v[5]), v[2], v[6], q16(v[3]), q16(v[7])};
  }
  __device__ static uint32_t vprep(uint32_t x) { return x; }
  // nibble pos (element pos; byte pos / 2, low nibble first) of dwords a and
  // b -> half2 of subnormals (a_pos, b_pos): byte pos / 2 of a and of b go to
  // bytes 0 and 2, whose low or high nibbles nib_lo / nib_hi convert.
  __device__ static h2_t vpair(uint32_t a, uint32_t b, int pos) {
    const uint32_t byte = (uint32_t)(pos >> 1);
    const uint32_t sel = 0x0C000C00u | ((4u + byte) << 16) | byte;
    const uint32_t t = __builtin_amdgcn_perm(b, a, sel);
    return (pos & 1) ? nib_hi(t) : nib_lo(t);
  }
};

// V-side operand of PV step c from the four exchanged chunks of a tile (lane
// (R, i) chunk j = token 4 R + j): slot k of the half4 = token 4 R + k,
// head-dim element VE * i + c.
template <int FMT, int D>
__device__ __forceinline__ h4_t vfrag(const uint32_t (&v)[4][VGeom<Fmt<FMT, D>::ROWB, D>::VD], int c) {
  using G = VGeom<Fmt<FMT, D>::ROWB, D>;
  const int dw = c / G::EPD;
  const int pos = c % G::EPD;
  const h2_t lo = Fmt<FMT, D>::vpair(v[0][dw], v[1][dw], pos);
  const h2_t hi = Fmt<FMT, D>::vpair(v[2][dw], v[3][dw], pos);
  return h4_t{lo.x, lo.y, hi.x, hi.y};
}

}  // namespace fqkv
