// gfx950 per-token KV quantizers: the on-GPU producers of the int8 / int4 KV
// formats the decode kernels read.
//
// Reference expressions (PyTorch, evaluated in the input's dtype):
//   int8: tests/test_kernels.py:32-34 -- s = max|x| / 127 clamped to >= 1e-8,
//         q = clamp(round(x / s), -127, 127), scales stored as fp16;
//   int4: nb:292-299 -- the same with 7, values packed two per byte, low
//         nibble = even element.
// The kernels reproduce those bytes exactly:
//   * the reference runs them on CUDA tensors, where PyTorch evaluates
//     a / qmax (tensor by Python scalar) as a * fp32(1/qmax), and x / s (tensor
//     by tensor) as a true division;
//   * fp32 input: s = max(a * fp32(1/qmax), 1e-8) and x / s in IEEE fp32
//     (correctly rounded division), round-half-even (v_rndne_f32), clamp,
//     scale = fp16(s);
//   * fp16 input: PyTorch evaluates each fp16 op in fp32 and rounds the result
//     to fp16, so s = fp16(a * fp32(1/qmax)) and every quotient is rounded to
//     fp16 before the round-half-even. A row whose fp16 scale underflows to 0 (max|x|
//     below ~4e-6) would divide by zero in the reference; here x = 0 maps to 0
//     and other x to +-qmax, the reference's clamp of +-inf.
//
// Layout: 16 lanes own one token row (D/16 consecutive elements each); a wave
// covers 4 rows per step, a 256-thread workgroup 16, grid-striding over rows.
// The append forms write a live cache's new K and V tokens in place, at host
// or device positions of contiguous caches, or at slots of paged caches.
// The row maximum is a DPP all-reduce within the 16-lane row. HBM-bound:
// reads 2 or 4 B per element, writes 1 or 0.5 B per element + 2 B per row.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "kv_formats.h"
#include "launch.h"

namespace fqkv {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// Max over each 16-lane row: quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror.
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f<0xB1>(x));
  x = fmaxf(x, dpp_f<0x4E>(x));
  x = fmaxf(x, dpp_f<0x141>(x));
  return fmaxf(x, dpp_f<0x140>(x));
}

// Source element types (the public header's FQKV_SRC_* values). bf16 rows
// widen exactly to fp32 and then follow the fp32 expressions.
enum { SRC_F16 = 0, SRC_F32 = 1, SRC_BF16 = 2 };
// the largest fp8 e4m3 value; as QMAX it selects the fp8 codes
constexpr int FP8_MAX = 448;

template <int SRC, int EPL>
__device__ __forceinline__ void load_row_slice(const void* X, int64_t row, int i, int D, float (&x)[EPL]) {
  if constexpr (SRC == SRC_BF16) {
    const uint16_t* p = (const uint16_t*)X + row * D + EPL * i;
    uint32_t w[EPL / 2];
    if constexpr (EPL == 8) {
      const u4_t v = *(const u4_t*)p;
      w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
    } else {
      const u2_t v = *(const u2_t*)p;
      w[0] = v.x, w[1] = v.y;
    }
#pragma unroll
    for (int k = 0; k < EPL / 2; ++k) {
      x[2 * k] = __builtin_bit_cast(float, w[k] << 16);
      x[2 * k + 1] = __builtin_bit_cast(float, w[k] & 0xFFFF0000u);
    }
  } else if constexpr (SRC == SRC_F16) {
    const _Float16* p = (const _Float16*)X + row * D + EPL * i;
    if constexpr (EPL == 8) {
      const h8_t v = *(const h8_t*)p;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 h = v[e];
        x[e] = (float)h;
      }
    } else {
      typedef _Float16 h4v_t __attribute__((ext_vector_type(4)));
      const h4v_t v = *(const h4v_t*)p;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 h = v[e];
        x[e] = (float)h;
      }
    }
  } else {
    const float* p = (const float*)X + row * D + EPL * i;
#pragma unroll
    for (int k = 0; k < EPL / 4; ++k) {
      const f4_t v = *(const f4_t*)(p + 4 * k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float f = v[e];
        x[4 * k + e] = f;
      }
    }
  }
}

// Quantize source row `row` of X into the destination row at qrow (D int8
// bytes or D/2 packed int4 bytes) and its scale at *srow. The calling 16
// lanes stay active together (the DPP reduction spans them); a group with
// live == false reads and writes nothing (its pointers may be anything).
template <int SRC, int QMAX, int D>
__device__ __forceinline__ void quantize_row(const void* __restrict__ X, int64_t row, uint8_t* __restrict__ qrow,
                                             _Float16* __restrict__ srow, bool live, int i) {
  // QMAX 448: fp8 e4m3 codes (no counterpart in the reference), always the
  // fp32 expressions: s = max(a * fp32(1/448), 1e-8), code = e4m3 round to
  // nearest even of clamp(x / s, +-448), scale stored as fp16(s)
  constexpr bool FP8 = QMAX == FP8_MAX;
  constexpr bool F16 = SRC == SRC_F16 && !FP8;  // fp16 rounding of the scale and the quotients
  constexpr int EPL = D / 16;  // elements per lane
  float x[EPL];
  if (live) {
    load_row_slice<SRC, EPL>(X, row, i, D, x);
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = 0.0f;
  }
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) a = fmaxf(a, fabsf(x[e]));
  a = row16_max(a);

  float s;          // the divisor, as the reference holds it
  _Float16 s_out;   // the stored scale
  if constexpr (F16) {
    s_out = (_Float16)(a * (1.0f / (float)QMAX));  // fp16 op: fp32 result rounded to fp16
    s = (float)s_out;                      // clamp(min=1e-8) cannot lift an fp16 value
  } else {
    s = fmaxf(a * (1.0f / (float)QMAX), 1e-8f);
    s_out = (_Float16)s;
  }
  // x / s as a true division rounds it, from one division per row: with
  // y = RN(1/s), q = RN(x y) and the exact residual r = x - q s (one FMA),
  // RN(q + r y) = RN(x / s) (Markstein's correction step). Checked against
  // the division for every fp16 x and every fp16 s, and on 1.6e9 random fp32
  // pairs with quotients at and next to the rounding ties; only the sign of
  // a zero quotient can differ, which rint and the int conversion drop.
  const float y = s != 0.0f ? 1.0f / s : 0.0f;
  auto divide = [&](float v) {
    const float q0 = v * y;
    return fmaf(fmaf(-q0, s, v), y, q0);
  };
  int q[EPL];
  float qf[FP8 ? EPL : 1];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    float quot;
    if constexpr (F16) {
      if (s == 0.0f) {
        quot = x[e] == 0.0f ? 0.0f : copysignf((float)QMAX, x[e]);
      } else {
        quot = (float)(_Float16)divide(x[e]);
      }
    } else {
      quot = divide(x[e]);
    }
    if constexpr (FP8) {
      qf[e] = fminf(fmaxf(quot, -(float)FP8_MAX), (float)FP8_MAX);
    } else {
      const float r = fminf(fmaxf(__builtin_rintf(quot), -(float)QMAX), (float)QMAX);
      q[e] = (int)r;
    }
  }
  if (!live) return;
  if constexpr (FP8) {
    // v_cvt_pk_fp8_f32 rounds to nearest even (OCP e4m3; the clamp keeps it
    // in range); two codes per call, into the low or the high half
    uint32_t w[EPL / 4];
#pragma unroll
    for (int k = 0; k < EPL / 4; ++k) {
      const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(qf[4 * k], qf[4 * k + 1], 0, false);
      w[k] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(qf[4 * k + 2], qf[4 * k + 3], lo, true);
    }
    uint8_t* out = qrow + EPL * i;
    if constexpr (EPL == 8) {
      *(u2_t*)out = u2_t{w[0], w[1]};
    } else {
      *(uint32_t*)out = w[0];
    }
  } else if constexpr (QMAX == 127) {
    uint32_t w[EPL / 4];
#pragma unroll
    for (int k = 0; k < EPL / 4; ++k)
      w[k] = (uint32_t)(q[4 * k] & 0xFF) | ((uint32_t)(q[4 * k + 1] & 0xFF) << 8) |
             ((uint32_t)(q[4 * k + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * k + 3] & 0xFF) << 24);
    uint8_t* out = qrow + EPL * i;
    if constexpr (EPL == 8) {
      *(u2_t*)out = u2_t{w[0], w[1]};
    } else {
      *(uint32_t*)out = w[0];
    }
  } else {
    uint32_t w = 0;
#pragma unroll
    for (int t = 0; t < EPL / 2; ++t)
      w |= ((uint32_t)(q[2 * t] & 0xF) | ((uint32_t)(q[2 * t + 1] & 0xF) << 4)) << (8 * t);
    uint8_t* out = qrow + (EPL / 2) * i;
    if constexpr (EPL == 8) {
      *(uint32_t*)out = w;
    } else {
      *(uint16_t*)out = (uint16_t)w;
    }
  }
  if (i == 0) *srow = s_out;
}

// Destination row dst of a contiguous [rows, D or D/2] code buffer.
template <int QMAX, int D>
__device__ __forceinline__ uint8_t* code_row(uint8_t* Q, int64_t dst) {
  return Q + dst * (QMAX == 7 ? D / 2 : D);
}

template <int SRC, int QMAX, int D>
__global__ void __launch_bounds__(256) quantize_kernel(const void* __restrict__ X, uint8_t* __restrict__ Q,
                                                       _Float16* __restrict__ scales, int64_t tokens) {
  const int i = threadIdx.x & 15;
  const int64_t rows_per_step = (int64_t)gridDim.x * (blockDim.x >> 4);
  for (int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4);
       row - (threadIdx.x >> 4) < tokens; row += rows_per_step)
    quantize_row<SRC, QMAX, D>(X, row, code_row<QMAX, D>(Q, row), scales + row, row < tokens, i);
}

// Append form for a live cache: K and V rows of `rows` cache rows x n new
// tokens ([rows, n, D] each, contiguous) go to token positions pos .. pos+n-1
// of caches laid out [rows, cap, D or D/2] with scales [rows, cap]. One launch
// covers both tensors: row index j < rows*n is K, the rest V. With pos_of set,
// the position of cache row r is pos_of[r / rows_per_pos] instead, read on the
// device (so a captured graph appends where the cache currently ends); rows
// whose tokens would not fit in [0, cap) are not written.
template <int SRC, int QMAX, int D>
__global__ void __launch_bounds__(256) quantize_append_kernel(const void* __restrict__ Xk, const void* __restrict__ Xv,
                                                              uint8_t* __restrict__ Qk, uint8_t* __restrict__ Qv,
                                                              _Float16* __restrict__ Sk, _Float16* __restrict__ Sv,
                                                              int64_t tokens, int64_t n, int64_t cap, int64_t pos,
                                                              const int32_t* __restrict__ pos_of, int64_t rows_per_pos) {
  const int i = threadIdx.x & 15;
  const int64_t rows_per_step = (int64_t)gridDim.x * (blockDim.x >> 4);
  for (int64_t j = (int64_t)blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4);
       j - (threadIdx.x >> 4) < 2 * tokens; j += rows_per_step) {
    const bool in = j < 2 * tokens;  // the same for the 16 lanes of a row
    const bool v = j >= tokens;
    const int64_t row = v ? j - tokens : j;
    const int64_t r = row / n;
    int64_t p = pos;
    bool fits = true;
    if (pos_of && in) {
      p = pos_of[r / rows_per_pos];
      fits = p >= 0 && p <= cap - n;
    }
    const int64_t dst = r * cap + (fits ? p : 0) + (row - r * n);
    quantize_row<SRC, QMAX, D>(v ? Xv : Xk, row, code_row<QMAX, D>(v ? Qv : Qk, dst), (v ? Sv : Sk) + dst, in && fits,
                               i);
  }
}

// Paged form for serving caches: token t's K and V rows ([tokens, heads, D]
// each, contiguous) go to cache slot slots[t] = page * page_size + offset of
// paged caches addressed by strides (codes in bytes, scales in elements), so
// token-major (NHD) and head-major (HND) pages take the same kernel. A slot
// outside [0, nslots) (a padding token, marked -1) writes nothing.
struct PagedDst {
  uint8_t* q[2];      // K, V codes
  _Float16* s[2];     // K, V scales
  int64_t q_page, q_tok, q_head;  // bytes
  int64_t s_page, s_tok, s_head;  // elements
  int64_t nslots;
  int page_log2;
};

template <int SRC, int QMAX, int D>
__global__ void __launch_bounds__(256) quantize_pages_kernel(const void* __restrict__ Xk, const void* __restrict__ Xv,
                                                             const int32_t* __restrict__ slots, int64_t rows,
                                                             int64_t heads, PagedDst d) {
  const int i = threadIdx.x & 15;
  const int64_t rows_per_step = (int64_t)gridDim.x * (blockDim.x >> 4);
  for (int64_t j = (int64_t)blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4);
       j - (threadIdx.x >> 4) < 2 * rows; j += rows_per_step) {
    const bool in = j < 2 * rows;  // the same for the 16 lanes of a row
    const int v = j >= rows ? 1 : 0;
    const int64_t row = v ? j - rows : j;  // token row * heads + head
    const int64_t t = row / heads;
    const int64_t h = row - t * heads;
    const int64_t slot = in ? (int64_t)slots[t] : -1;
    const bool live = slot >= 0 && slot < d.nslots;
    const int64_t pg = live ? slot >> d.page_log2 : 0;
    const int64_t off = live ? slot - (pg << d.page_log2) : 0;
    quantize_row<SRC, QMAX, D>(v ? Xv : Xk, row, d.q[v] + pg * d.q_page + off * d.q_tok + h * d.q_head,
                               d.s[v] + pg * d.s_page + off * d.s_tok + h * d.s_head, live, i);
  }
}

template <int SRC, int QMAX>
hipError_t launch_qp(int D, const void* Xk, const void* Xv, const int32_t* slots, int64_t rows, int64_t heads,
                     const PagedDst& d, hipStream_t st) {
  const int64_t want = (2 * rows + 15) / 16;
  const unsigned grid = (unsigned)(want < (1 << 16) ? want : (1 << 16));
  if (D == 128)
    hipLaunchKernelGGL((quantize_pages_kernel<SRC, QMAX, 128>), dim3(grid), dim3(256), 0, st, Xk, Xv, slots, rows,
                       heads, d);
  else
    hipLaunchKernelGGL((quantize_pages_kernel<SRC, QMAX, 64>), dim3(grid), dim3(256), 0, st, Xk, Xv, slots, rows,
                       heads, d);
  return hipGetLastError();
}

template <int SRC, int QMAX>
hipError_t launch_q(int D, const void* X, void* Q, void* S, int64_t tokens, hipStream_t st) {
  const int64_t want = (tokens + 15) / 16;
  const unsigned grid = (unsigned)(want < (1 << 16) ? want : (1 << 16));
  if (D == 128)
    hipLaunchKernelGGL((quantize_kernel<SRC, QMAX, 128>), dim3(grid), dim3(256), 0, st, X, (uint8_t*)Q,
                       (_Float16*)S, tokens);
  else
    hipLaunchKernelGGL((quantize_kernel<SRC, QMAX, 64>), dim3(grid), dim3(256), 0, st, X, (uint8_t*)Q,
                       (_Float16*)S, tokens);
  return hipGetLastError();
}

template <int SRC, int QMAX>
hipError_t launch_qa(int D, const void* Xk, const void* Xv, void* Qk, void* Qv, void* Sk, void* Sv, int64_t tokens,
                     int64_t n, int64_t cap, int64_t pos, const int32_t* pos_of, int64_t rows_per_pos,
                     hipStream_t st) {
  const int64_t want = (2 * tokens + 15) / 16;
  const unsigned grid = (unsigned)(want < (1 << 16) ? want : (1 << 16));
  if (D == 128)
    hipLaunchKernelGGL((quantize_append_kernel<SRC, QMAX, 128>), dim3(grid), dim3(256), 0, st, Xk, Xv,
                       (uint8_t*)Qk, (uint8_t*)Qv, (_Float16*)Sk, (_Float16*)Sv, tokens, n, cap, pos, pos_of,
                       rows_per_pos);
  else
    hipLaunchKernelGGL((quantize_append_kernel<SRC, QMAX, 64>), dim3(grid), dim3(256), 0, st, Xk, Xv,
                       (uint8_t*)Qk, (uint8_t*)Qv, (_Float16*)Sk, (_Float16*)Sv, tokens, n, cap, pos, pos_of,
                       rows_per_pos);
  return hipGetLastError();
}

}  // namespace

// A launcher templated on <SRC, QMAX> for run-time source type and format.
template <typename Fn>
hipError_t by_src_fmt(int src, int fmt, Fn f) {
  auto q = [&](auto src_c) -> hipError_t {
    if (fmt == KV_I8) return f(src_c, std::integral_constant<int, 127>());
    if (fmt == KV_I4) return f(src_c, std::integral_constant<int, 7>());
    if (fmt == KV_FP8) return f(src_c, std::integral_constant<int, FP8_MAX>());
    return hipErrorInvalidValue;
  };
  switch (src) {
    case SRC_F16: return q(std::integral_constant<int, SRC_F16>());
    case SRC_F32: return q(std::integral_constant<int, SRC_F32>());
    case SRC_BF16: return q(std::integral_constant<int, SRC_BF16>());
  }
  return hipErrorInvalidValue;
}

hipError_t launch_quantize_append(int src, int fmt, int D, const void* Xk, const void* Xv, void* Qk, void* Qv,
                                  void* Sk, void* Sv, int64_t rows, int64_t n, int64_t cap, int64_t pos,
                                  const int32_t* pos_of, int64_t rows_per_pos, hipStream_t st) {
  if (rows < 1 || n < 1 || cap < 1 || n > cap || (D != 64 && D != 128)) return hipErrorInvalidValue;
  if (pos_of ? (rows_per_pos < 1 || rows % rows_per_pos != 0) : (pos < 0 || pos + n > cap))
    return hipErrorInvalidValue;
  const int64_t tokens = rows * n;
  return by_src_fmt(src, fmt, [&](auto s_c, auto q_c) {
    return launch_qa<decltype(s_c)::value, decltype(q_c)::value>(D, Xk, Xv, Qk, Qv, Sk, Sv, tokens, n, cap, pos,
                                                                  pos_of, rows_per_pos, st);
  });
}

hipError_t launch_quantize_pages(int src, int fmt, int D, const void* Xk, const void* Xv, const int32_t* slots,
                                 int64_t tokens, int64_t heads, void* Qk, void* Qv, void* Sk, void* Sv,
                                 int64_t num_pages, int page_log2, int64_t q_page, int64_t q_tok, int64_t q_head,
                                 int64_t s_page, int64_t s_tok, int64_t s_head, hipStream_t st) {
  if (tokens < 1 || heads < 1 || num_pages < 1 || page_log2 < 0 || page_log2 > 30 || (D != 64 && D != 128))
    return hipErrorInvalidValue;
  PagedDst d;
  d.q[0] = (uint8_t*)Qk;
  d.q[1] = (uint8_t*)Qv;
  d.s[0] = (_Float16*)Sk;
  d.s[1] = (_Float16*)Sv;
  d.q_page = q_page;
  d.q_tok = q_tok;
  d.q_head = q_head;
  d.s_page = s_page;
  d.s_tok = s_tok;
  d.s_head = s_head;
  d.nslots = num_pages << page_log2;
  d.page_log2 = page_log2;
  const int64_t rows = tokens * heads;
  return by_src_fmt(src, fmt, [&](auto s_c, auto q_c) {
    return launch_qp<decltype(s_c)::value, decltype(q_c)::value>(D, Xk, Xv, slots, rows, heads, d, st);
  });
}

hipError_t launch_quantize(int src, int fmt, int D, const void* X, void* Q, void* S, int64_t tokens,
                           hipStream_t st) {
  if (tokens < 1 || (D != 64 && D != 128)) return hipErrorInvalidValue;
  return by_src_fmt(src, fmt, [&](auto s_c, auto q_c) {
    return launch_q<decltype(s_c)::value, decltype(q_c)::value>(D, X, Q, S, tokens, st);
  });
}

}  // namespace fqkv
