// gfx950 kernels of the fused single-query decode-attention path.
//
// One partial kernel serves all five entry points. A workgroup owns one
// (KV row r, query-head group, split s) work item: it streams the split's
// K/V token range of KV row r exactly once and applies it to up to HG query
// heads of that row (HG = 1 for MHA; the GQA group for GQA), so compact GQA
// KV is read once per group instead of once per query head. Waves take
// interleaved 16-token tiles in passes of U tiles: a pass first issues every
// load of its U tiles (raw buffer loads from a descriptor that ends at the
// split's last token, so rows past it read as zeros and need no clamping),
// then consumes the tiles in order while the later ones are still arriving.
// Per tile a wave
//   1. has loaded the K tile as matrix-core operand B (dwordx4, 64 contiguous
//      bytes per row per instruction) and the V tile as 16-byte row slices,
//   2. computes all HG x 16 scores with D/32 v_mfma_f32_16x16x32_f16 (query
//      head slots on the M axis, tokens on N),
//   3. runs one online-softmax step per 16-lane row (= one head) with DPP
//      row reductions and v_exp_f32 (exp(x) = 2^(x log2 e), log2 e folded
//      into the score scale),
//   4. hands the per-token weights to the V lanes through a wave-private LDS
//      slot and accumulates p * V in fp32 registers.
// Waves of a workgroup take interleaved tiles; their (m, l, acc) states are
// merged through LDS. With one split the workgroup writes the normalised
// fp16 output; otherwise it writes the reference's fp32 scratch layout
// (m_part[h*S+s], l_part[h*S+s], o_part[(h*S+s)*D+d]) and the combine
// kernel merges the splits.
//
// Reference algorithm: decode_attn_gqa_sk_fast.cu:6-54 (partial),
// :57-94 (combine); decode_attn_fp16_mw.cu:6-49 and decode_attn_gqa.cu:8-55
// are the single-split case; decode_attn_int8_mw.cu:6-51 and
// decode_attn_int4.cu:8-46 add per-token scales.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kv_formats.h"
#include "launch.h"

namespace fqkv {

constexpr float LOG2E = 1.4426950408889634f;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// All-reduce over each 16-lane row: quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror.
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  return x;
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  return x;
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
__device__ __forceinline__ void compiler_fence() { __asm__ __volatile__("" ::: "memory"); }

template <int FMT, int D, int HG>
__global__ void __launch_bounds__(64 * NW_MAX) decode_partial_kernel(PartialParams p) {
  using F = Fmt<FMT, D>;
  constexpr int U = 4;
  constexpr int NR = (HG + 3) / 4;  // MFMA result registers that carry heads
  __shared__ float s_w[NW_MAX][16][HG];
  __shared__ float s_o[NW_MAX][HG][D];
  __shared__ float s_m[NW_MAX][HG];
  __shared__ float s_l[NW_MAX][HG];

  const int lane = threadIdx.x & 63;
  // wave index as a scalar, so tile loops branch per wave, not per lane
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  int wg = blockIdx.x;
  const int s = wg % p.S;
  wg /= p.S;
  const int hg = wg % p.ngroups;
  const int r = wg / p.ngroups;
  const int lo = s * p.chunk;
  const int hi = min(lo + p.chunk, p.N);
  const int hbase = hg * HG;
  const int hcnt = min(HG, p.G - hbase);
  const size_t qrow0 = (size_t)r * p.G + hbase;
  const uint8_t* Kr = p.K + (size_t)r * p.N * F::ROWB;
  const uint8_t* Vr = p.V + (size_t)r * p.N * F::ROWB;
  const _Float16* Ksr = F::QUANT ? p.Ks + (size_t)r * p.N : nullptr;
  const _Float16* Vsr = F::QUANT ? p.Vs + (size_t)r * p.N : nullptr;

  const int kt = lane & 15;  // token of the tile this lane scores
  const int kb = lane >> 4;  // K dword group / head-slot group
  const int vl = lane % F::LPR;
  const int vt = lane / F::LPR;

  // Query fragment (MFMA operand A). Row m = lane % 16 carries head slot
  // 4 (m % 4) + m / 4, so result register rr of lane l holds head (l / 16) + 4 rr.
  // The descriptor covers only this group's hcnt query rows: slots past them
  // read as zeros and score nothing.
  h8_t qa[F::NKI];
  {
    const int m = lane & 15;
    const int h = 4 * (m & 3) + (m >> 2);
    const rsrc_t rQ = make_rsrc(p.q + qrow0 * D, (uint32_t)hcnt * D * 2);
#pragma unroll
    for (int i = 0; i < F::NKI; ++i) qa[i] = F::qfrag(rQ, (uint32_t)h * D, i, kb);
  }

  float m_run[NR], l_run[NR], c_run[NR];
#pragma unroll
  for (int rr = 0; rr < NR; ++rr) {
    m_run[rr] = -INFINITY;
    l_run[rr] = 0.0f;
    c_run[rr] = 0.0f;
  }
  float acc[HG][F::EV];
#pragma unroll
  for (int h = 0; h < HG; ++h)
#pragma unroll
    for (int e = 0; e < F::EV; ++e) acc[h][e] = 0.0f;

  struct Tile {
    typename F::KT kr[F::KL];
    vraw_t<F::VB> vr[F::VLD];
    float ksc, vsc;
  };
  // Buffer descriptors end at the split's last token, so rows past it read
  // as zeros (their scores are masked); offsets are 32-bit from the row block.
  const uint32_t nbytes = (uint32_t)hi * F::ROWB;
  const rsrc_t rK = make_rsrc(Kr, nbytes);
  const rsrc_t rV = make_rsrc(Vr, nbytes);
  const rsrc_t rKs = make_rsrc(Ksr, 2u * (uint32_t)hi);
  const rsrc_t rVs = make_rsrc(Vsr, 2u * (uint32_t)hi);
  const uint32_t koff = (uint32_t)kt * F::ROWB + F::klane(kb);
  const uint32_t voff = (uint32_t)vt * F::ROWB + (uint32_t)vl * F::VB;
  auto load_tile = [&](Tile& t, int tb) {
    const uint32_t base = (uint32_t)tb * F::ROWB;
    F::load_k(rK, base + koff, t.kr);
    if constexpr (F::QUANT) {
      t.ksc = (float)__builtin_bit_cast(_Float16, buf_load<2>(rKs, 2u * (uint32_t)(tb + kt)));
      t.vsc = (float)__builtin_bit_cast(_Float16, buf_load<2>(rVs, 2u * (uint32_t)(tb + kt)));
    } else {
      t.ksc = 1.0f;
      t.vsc = 1.0f;
    }
#pragma unroll
    for (int j = 0; j < F::VLD; ++j) t.vr[j] = load_v<FMT, D>(rV, base + voff + (uint32_t)(j * F::TPL * F::ROWB));
  };
  // Scores, online-softmax step and p*V accumulation for one loaded tile.
  auto process_tile = [&](const Tile& t, int tb) {
    f4_t c4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < F::NKI; ++i)
      c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[i], F::kfrag(t.kr, i), c4, 0, 0, 0);
    const bool tok_ok = tb + kt < hi;
    float alpha[NR];
#pragma unroll
    for (int rr = 0; rr < NR; ++rr) {
      const int h = kb + 4 * rr;
      float x = c4[rr] * t.ksc;
      x = (tok_ok && h < hcnt) ? x : -INFINITY;
      const float mn = fmaxf(m_run[rr], row16_max(x));
      const float mu = (mn == -INFINITY) ? 0.0f : mn;
      alpha[rr] = fast_exp2((m_run[rr] - mu) * p.c);
      const float pw = fast_exp2((x - mu) * p.c);
      l_run[rr] = l_run[rr] * alpha[rr] + pw;
      const float wv = pw * t.vsc;
      if constexpr (F::QUANT) c_run[rr] = c_run[rr] * alpha[rr] + wv;
      m_run[rr] = mn;
      if (h < HG) s_w[w][kt][h] = wv;
    }
    compiler_fence();
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      const float a = readlane_f(alpha[h / 4], 16 * (h % 4));
      if (a != 1.0f) {
#pragma unroll
        for (int e = 0; e < F::EV; ++e) acc[h][e] *= a;
      }
    }
#pragma unroll
    for (int j = 0; j < F::VLD; ++j) {
      const int tl = j * F::TPL + vt;
      float wt[HG];
#pragma unroll
      for (int h = 0; h < HG; ++h) wt[h] = s_w[w][tl][h];
      float f[F::EV];
      F::vconv(t.vr[j], f);
#pragma unroll
      for (int h = 0; h < HG; ++h)
#pragma unroll
        for (int e = 0; e < F::EV; ++e) acc[h][e] = fmaf(wt[h], f[e], acc[h][e]);
    }
    compiler_fence();
  };

  // Two-tile register pipeline: the next tile's loads are in flight while the
  // current tile is processed. Every branch below is wave-uniform, and each
  // path either prefetches before processing or processes the last tile, so
  // the compiler's load counters wait only for the tile being consumed.
  // Each pass a wave issues the loads of U tiles (interleaved with the other
  // waves' tiles) before consuming any: straight-line code, so the load
  // counter waits exactly for the tile about to be used while the rest of the
  // pass is still in flight. Tiles past the split end are clamped and masked.
  const int step = 16 * nw;
  for (int pb = lo + 16 * w; pb < hi; pb += U * step) {
    Tile t[U];
#pragma unroll
    for (int u = 0; u < U; ++u) load_tile(t[u], pb + u * step);
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the pass ahead of its use
#pragma unroll
    for (int u = 0; u < U; ++u) process_tile(t[u], pb + u * step);
  }

  // ---- wave totals ----
#pragma unroll
  for (int rr = 0; rr < NR; ++rr) {
    l_run[rr] = row16_sum(l_run[rr]);
    if constexpr (F::QUANT) c_run[rr] = row16_sum(c_run[rr]);
  }
#pragma unroll
  for (int h = 0; h < HG; ++h)
#pragma unroll
    for (int e = 0; e < F::EV; ++e) {
      float v = acc[h][e];
#pragma unroll
      for (int x = F::LPR; x < 64; x <<= 1) v += __shfl_xor(v, x);
      acc[h][e] = v;
    }
  if constexpr (F::QUANT) {
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      const float cw = readlane_f(c_run[h / 4], 16 * (h % 4));
#pragma unroll
      for (int e = 0; e < F::EV; ++e) acc[h][e] -= F::VBIAS * cw;
    }
  }
  if (lane < F::LPR) {
#pragma unroll
    for (int h = 0; h < HG; ++h)
#pragma unroll
      for (int e = 0; e < F::EV; ++e) s_o[w][h][F::vd_index(lane, e)] = acc[h][e];
  }
  if (kt == 0) {
#pragma unroll
    for (int rr = 0; rr < NR; ++rr) {
      const int h = kb + 4 * rr;
      if (h < HG) {
        s_m[w][h] = m_run[rr];
        s_l[w][h] = l_run[rr];
      }
    }
  }
  __syncthreads();

  // ---- merge the waves, emit output or split scratch ----
  for (int idx = threadIdx.x; idx < hcnt * D; idx += blockDim.x) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = -INFINITY;
    for (int ww = 0; ww < nw; ++ww) M = fmaxf(M, s_m[ww][h]);
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
      for (int ww = 0; ww < nw; ++ww) {
        const float sc = fast_exp2((s_m[ww][h] - M) * p.c);
        L += sc * s_l[ww][h];
        O += sc * s_o[ww][h][d];
      }
    }
    const size_t qh = qrow0 + h;
    if (p.direct) {
      p.o[qh * D + d] = (_Float16)(O / L);
    } else {
      const size_t b = qh * p.S + s;
      if (d == 0) {
        p.m_part[b] = (M == -INFINITY) ? -INFINITY : M * p.scale;
        p.l_part[b] = L;
      }
      p.o_part[b * D + d] = O;
    }
  }
}

// Merge S split partials of one query head per workgroup:
// o = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s (decode_attn_gqa_sk_fast.cu:57-94).
// Every thread first reduces M; wave w then takes splits w, w + nw, ...
// with lanes covering the head dimension (D/64 floats each); waves meet in LDS.
template <int D>
__global__ void __launch_bounds__(64 * NW_MAX) combine_kernel(const float* __restrict__ m_part,
                                                              const float* __restrict__ l_part,
                                                              const float* __restrict__ o_part,
                                                              _Float16* __restrict__ o, int S) {
  constexpr int E = D / 64;
  __shared__ float s_red[NW_MAX];
  __shared__ float s_l[NW_MAX];
  __shared__ float s_o[NW_MAX][D];
  const int h = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const float* mh = m_part + (size_t)h * S;
  const float* lh = l_part + (size_t)h * S;
  const float* oh = o_part + (size_t)h * S * D;

  float M = -INFINITY;
  for (int s = threadIdx.x; s < S; s += blockDim.x) M = fmaxf(M, mh[s]);
#pragma unroll
  for (int x = 32; x > 0; x >>= 1) M = fmaxf(M, __shfl_xor(M, x));
  if (lane == 0) s_red[w] = M;
  __syncthreads();
  M = -INFINITY;
  for (int ww = 0; ww < nw; ++ww) M = fmaxf(M, s_red[ww]);

  float L = 0.0f, O[E];
#pragma unroll
  for (int e = 0; e < E; ++e) O[e] = 0.0f;
  if (M != -INFINITY) {
    for (int s = w; s < S; s += nw) {
      const float sc = fast_exp2((mh[s] - M) * LOG2E);  // empty split: m = -inf -> 0
      L += sc * lh[s];
      const float* src = oh + (size_t)s * D + lane * E;
#pragma unroll
      for (int e = 0; e < E; ++e) O[e] += sc * src[e];
    }
  }
  if (lane == 0) s_l[w] = L;
#pragma unroll
  for (int e = 0; e < E; ++e) s_o[w][lane * E + e] = O[e];
  __syncthreads();
  if (w == 0) {
    float Lt = 0.0f;
    for (int ww = 0; ww < nw; ++ww) Lt += s_l[ww];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float Ot = 0.0f;
      for (int ww = 0; ww < nw; ++ww) Ot += s_o[ww][lane * E + e];
      o[(size_t)h * D + lane * E + e] = (_Float16)(Ot / Lt);
    }
  }
}

// Dequantise through the kernels' own conversions (K side: int -> fp16
// operand; V side: int -> fp32 plus bias), one thread per (token, lane slot).
template <int FMT, int D>
__global__ void dequant_kernel(const uint8_t* __restrict__ Kq, const _Float16* __restrict__ Ks,
                               float* __restrict__ out, int64_t tokens, int path) {
  using F = Fmt<FMT, D>;
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (path == 0) {
    const int64_t t = g / 4;
    const int kb = (int)(g % 4);
    if (t >= tokens) return;
    typename F::KT kr[F::KL];
    F::load_k(make_rsrc(Kq + t * F::ROWB, F::ROWB), F::klane(kb), kr);
    const float sc = (float)Ks[t];
#pragma unroll
    for (int i = 0; i < F::NKI; ++i) {
      const h8_t b = F::kfrag(kr, i);
#pragma unroll
      for (int e = 0; e < 8; ++e) out[t * D + F::kd_index(i, kb, e)] = (float)b[e] * sc;
    }
  } else {
    const int64_t t = g / F::LPR;
    const int lir = (int)(g % F::LPR);
    if (t >= tokens) return;
    float f[F::EV];
    F::vconv(load_v<FMT, D>(make_rsrc(Kq + t * F::ROWB, F::ROWB), (uint32_t)lir * F::VB), f);
    const float sc = (float)Ks[t];
#pragma unroll
    for (int e = 0; e < F::EV; ++e) out[t * D + F::vd_index(lir, e)] = (f[e] - F::VBIAS) * sc;
  }
}

// ------------------------------------------------------------ launchers ----
template <int FMT, int D, int HG>
static hipError_t launch_partial_t(const PartialParams& p, int nblocks, int nw, hipStream_t st) {
  hipLaunchKernelGGL((decode_partial_kernel<FMT, D, HG>), dim3(nblocks), dim3(64 * nw), 0, st, p);
  return hipGetLastError();
}

template <int FMT, int D>
static hipError_t launch_partial_d(int hg, const PartialParams& p, int nblocks, int nw, hipStream_t st) {
  if constexpr (FMT == KV_F16) {
    switch (hg) {
      case 1: return launch_partial_t<FMT, D, 1>(p, nblocks, nw, st);
      case 2: return launch_partial_t<FMT, D, 2>(p, nblocks, nw, st);
      case 4: return launch_partial_t<FMT, D, 4>(p, nblocks, nw, st);
      case 8: return launch_partial_t<FMT, D, 8>(p, nblocks, nw, st);
    }
  } else {
    if (hg == 1) return launch_partial_t<FMT, D, 1>(p, nblocks, nw, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_partial(int fmt, int D, int hg, const PartialParams& p, int nblocks, int nw,
                          hipStream_t st) {
  if (nw < 1 || nw > NW_MAX || nblocks < 1) return hipErrorInvalidValue;
  switch (fmt) {
    case KV_F16: return D == 64 ? launch_partial_d<KV_F16, 64>(hg, p, nblocks, nw, st)
                                : launch_partial_d<KV_F16, 128>(hg, p, nblocks, nw, st);
    case KV_I8: return D == 64 ? launch_partial_d<KV_I8, 64>(hg, p, nblocks, nw, st)
                               : launch_partial_d<KV_I8, 128>(hg, p, nblocks, nw, st);
    case KV_I4: return D == 64 ? launch_partial_d<KV_I4, 64>(hg, p, nblocks, nw, st)
                               : launch_partial_d<KV_I4, 128>(hg, p, nblocks, nw, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_combine(int D, const float* m_part, const float* l_part, const float* o_part,
                          void* o, int H, int S, int nw, hipStream_t st) {
  if (nw < 1 || nw > NW_MAX || H < 1 || S < 1) return hipErrorInvalidValue;
  if (D == 64)
    hipLaunchKernelGGL((combine_kernel<64>), dim3(H), dim3(64 * nw), 0, st, m_part, l_part, o_part,
                       (_Float16*)o, S);
  else
    hipLaunchKernelGGL((combine_kernel<128>), dim3(H), dim3(64 * nw), 0, st, m_part, l_part, o_part,
                       (_Float16*)o, S);
  return hipGetLastError();
}

hipError_t launch_dequant(int fmt, int D, int path, const void* Kq, const void* Ks, float* out,
                          int64_t tokens, hipStream_t st) {
  const int lpr = (fmt == KV_I8) ? (D == 128 ? Fmt<KV_I8, 128>::LPR : Fmt<KV_I8, 64>::LPR)
                                 : (D == 128 ? Fmt<KV_I4, 128>::LPR : Fmt<KV_I4, 64>::LPR);
  const int64_t threads = tokens * (path == 0 ? 4 : lpr);
  const int64_t blocks = (threads + 255) / 256;
  const auto* k = (const uint8_t*)Kq;
  const auto* s = (const _Float16*)Ks;
  if (fmt == KV_I8) {
    if (D == 128)
      hipLaunchKernelGGL((dequant_kernel<KV_I8, 128>), dim3(blocks), dim3(256), 0, st, k, s, out, tokens, path);
    else
      hipLaunchKernelGGL((dequant_kernel<KV_I8, 64>), dim3(blocks), dim3(256), 0, st, k, s, out, tokens, path);
  } else if (fmt == KV_I4) {
    if (D == 128)
      hipLaunchKernelGGL((dequant_kernel<KV_I4, 128>), dim3(blocks), dim3(256), 0, st, k, s, out, tokens, path);
    else
      hipLaunchKernelGGL((dequant_kernel<KV_I4, 64>), dim3(blocks), dim3(256), 0, st, k, s, out, tokens, path);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace fqkv
