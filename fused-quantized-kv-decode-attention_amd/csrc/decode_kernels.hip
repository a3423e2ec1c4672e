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
// Sum of x over the lanes of the wave that share (lane % LPR): rotations
// within each 16-lane row for LPR < 16, then v_permlane16_swap (rows 0+1,
// 2+3) and v_permlane32_swap (halves). Adding both swap outputs makes the
// result independent of which operand receives which half. All VALU.
template <int LPR>
__device__ __forceinline__ float sum_over_token_rows(float x) {
  if constexpr (LPR <= 4) x += dpp<0x124>(x);  // row_ror:4
  if constexpr (LPR <= 8) x += dpp<0x128>(x);  // row_ror:8
  // (swap results are copied to scalars before the bit casts: this
  // compiler's __builtin_bit_cast of a vector element reads element 0)
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const unsigned a = r16[0], b = r16[1];
  x = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  const unsigned v = __builtin_bit_cast(unsigned, x);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  const unsigned c = r32[0], d = r32[1];
  return __builtin_bit_cast(float, c) + __builtin_bit_cast(float, d);
}
__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
__device__ __forceinline__ void compiler_fence() { __asm__ __volatile__("" ::: "memory"); }

typedef float fl4_t __attribute__((ext_vector_type(4)));

// Arrival counters of the in-kernel split merge. Zero at load; the workgroup
// that merges a group resets its counter, so every call leaves them at zero.
__device__ int g_split_arrivals[SPLIT_SLOTS][MAX_SPLIT_GROUPS];

// Merge S split partials for query heads h0 .. h0+nh-1 with the whole
// workgroup: o[h] = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s
// (decode_attn_gqa_sk_fast.cu:57-94; m in natural-log units, an empty split
// has m = -inf and weight 0). Thread t owns float4 column c of head hh for
// splits g, g + NG, ...; it issues a chunk of CH splits' loads before the
// block-wide maximum is known, so a merge costs about one memory round trip.
// s_acc holds blockDim.x float4, s_red 2 * blockDim.x / (D/4) floats.
// COHERENT: read the partials with device-scope (sc1) loads, for partials
// that other workgroups of the same launch stored with device-scope stores.
template <int D, bool COHERENT>
__device__ void merge_splits(const float* __restrict__ m_part, const float* __restrict__ l_part,
                             const float* __restrict__ o_part, _Float16* __restrict__ o, size_t h0,
                             int nh, int S, fl4_t* s_acc, float* s_red) {
  constexpr int C4 = D / 4;
  constexpr int CH = 8;
  auto ld1 = [](const float* ptr) -> float {
    if constexpr (COHERENT) return __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *ptr;
  };
  // one descriptor (uniform) over the acc partials of heads h0 .. h0+nh-1
  const rsrc_t rO = make_rsrc(o_part + h0 * S * D, (uint32_t)(nh * S * D) * 4u);
  auto ld4 = [&](const fl4_t* base, uint32_t idx) -> fl4_t {
    if constexpr (COHERENT) {
      const uint32_t off = (uint32_t)((const float*)(base + idx) - (o_part + h0 * S * D)) * 4u;
      return __builtin_bit_cast(fl4_t, __builtin_amdgcn_raw_buffer_load_b128(rO, (int)off, 0, CPOL_SC1));
    } else {
      return base[idx];
    }
  };
  const int t = threadIdx.x;
  const int nt = blockDim.x;
  const int hpr = nt / C4;  // heads per round (>= 4: nt >= 128, C4 <= 32)
  float* s_mx = s_red;
  float* s_l = s_red + hpr;
  for (int hb = 0; hb < nh; hb += hpr) {
    const int hr = min(hpr, nh - hb);
    const int NG = nt / (C4 * hr);
    const int c = t % C4;
    const int hh = (t / C4) % hr;
    const int g = t / (C4 * hr);
    const bool act = g < NG;
    const size_t h = h0 + hb + hh;
    const float* mh = m_part + h * S;
    const float* lh = l_part + h * S;
    const fl4_t* oh = reinterpret_cast<const fl4_t*>(o_part + h * S * D);
    fl4_t ov[CH];
    float mv[CH], lv[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const int sk = g + k * NG;
      const bool ok = act && sk < S;
      ov[k] = ok ? ld4(oh, (uint32_t)(sk * C4 + c)) : fl4_t{0.0f, 0.0f, 0.0f, 0.0f};
      mv[k] = ok ? ld1(mh + sk) : -INFINITY;
      lv[k] = ok ? ld1(lh + sk) : 0.0f;
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int k = 0; k < CH; ++k) mloc = fmaxf(mloc, mv[k]);
    if (act)
      for (int sk = g + CH * NG; sk < S; sk += NG) mloc = fmaxf(mloc, ld1(mh + sk));
    if (act && c == 0) s_mx[g * hr + hh] = mloc;
    __syncthreads();
    float M = -INFINITY;
    for (int gg = 0; gg < NG; ++gg) M = fmaxf(M, s_mx[gg * hr + hh]);
    fl4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float L = 0.0f;
    if (act && M != -INFINITY) {
      for (int base = 0;; base += CH * NG) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const float sc = fast_exp2((mv[k] - M) * LOG2E);
          L += sc * lv[k];
          acc += sc * ov[k];
        }
        const int nb = base + CH * NG;
        if (nb >= S) break;
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const int sk = nb + g + k * NG;
          const bool ok = sk < S;
          ov[k] = ok ? ld4(oh, (uint32_t)(sk * C4 + c)) : fl4_t{0.0f, 0.0f, 0.0f, 0.0f};
          mv[k] = ok ? ld1(mh + sk) : -INFINITY;
          lv[k] = ok ? ld1(lh + sk) : 0.0f;
        }
      }
    }
    s_acc[t] = acc;
    if (act && c == 0) s_l[g * hr + hh] = L;
    __syncthreads();
    if (t < hr * C4) {
      const int oh2 = t / C4;
      const int c2 = t % C4;
      fl4_t r = {0.0f, 0.0f, 0.0f, 0.0f};
      float Lt = 0.0f;
      for (int gg = 0; gg < NG; ++gg) {
        r += s_acc[(gg * hr + oh2) * C4 + c2];
        Lt += s_l[gg * hr + oh2];
      }
      r /= Lt;
      _Float16* dst = o + (h0 + hb + oh2) * D + 4 * c2;
      dst[0] = (_Float16)r.x;
      dst[1] = (_Float16)r.y;
      dst[2] = (_Float16)r.z;
      dst[3] = (_Float16)r.w;
    }
    __syncthreads();
  }
}

template <int FMT, int D, int HG>
__global__ void __launch_bounds__(64 * NW_MAX) decode_partial_kernel(PartialParams p) {
  using F = Fmt<FMT, D>;
  constexpr int U = 4;
  constexpr int NR = (HG + 3) / 4;  // MFMA result registers that carry heads
  __shared__ float s_w[NW_MAX][U][16][HG];
  __shared__ float s_o[NW_MAX][HG][D];
  __shared__ float s_m[HG][NW_MAX];
  __shared__ float s_l[HG][NW_MAX];
  __shared__ fl4_t s_macc[64 * NW_MAX];        // in-kernel split merge
  __shared__ float s_mred[2 * 64 * NW_MAX / (D / 4)];
  __shared__ int s_last;

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

  // Buffer descriptors end at the split's last token, so rows past it read
  // as zeros (their scores are masked); offsets are 32-bit from the row block.
  const uint32_t nbytes = (uint32_t)hi * F::ROWB;
  const rsrc_t rK = make_rsrc(Kr, nbytes);
  const rsrc_t rV = make_rsrc(Vr, nbytes);
  const rsrc_t rKs = make_rsrc(Ksr, 2u * (uint32_t)hi);
  const rsrc_t rVs = make_rsrc(Vsr, 2u * (uint32_t)hi);
  const uint32_t koff = (uint32_t)kt * F::ROWB + F::klane(kb);
  const uint32_t voff = (uint32_t)vt * F::ROWB + (uint32_t)vl * F::VB;

  // Each pass covers U tiles of this wave (tiles interleave across waves).
  // All K loads of the pass are issued, then all V loads, before anything is
  // consumed: straight-line code, so the load counter waits exactly for the
  // data about to be used while the rest is still arriving. The pass then
  // scores all U tiles with the matrix cores, takes ONE online-softmax step
  // over its 16 U tokens per row (one max reduction, one rescale), and
  // accumulates p * V.
  const int step = 16 * nw;
  for (int pb = lo + 16 * w; pb < hi; pb += U * step) {
    typename F::KT kr[U][F::KL];
    vraw_t<F::VB> vr[U][F::VLD];
    float ksc[U], vsc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t base = (uint32_t)(pb + u * step) * F::ROWB;
      F::load_k(rK, base + koff, kr[u]);
      if constexpr (F::QUANT) {
        const uint32_t so = 2u * (uint32_t)(pb + u * step + kt);
        ksc[u] = (float)__builtin_bit_cast(_Float16, buf_load<2>(rKs, so));
        vsc[u] = (float)__builtin_bit_cast(_Float16, buf_load<2>(rVs, so));
      } else {
        ksc[u] = 1.0f;
        vsc[u] = 1.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t base = (uint32_t)(pb + u * step) * F::ROWB;
#pragma unroll
      for (int j = 0; j < F::VLD; ++j) vr[u][j] = load_v<FMT, D>(rV, base + voff + (uint32_t)(j * F::TPL * F::ROWB));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the pass ahead of its use

    f4_t c4[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      c4[u] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < F::NKI; ++i)
        c4[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[i], F::kfrag(kr[u], i), c4[u], 0, 0, 0);
    }

    float alpha[NR];
#pragma unroll
    for (int rr = 0; rr < NR; ++rr) {
      const int h = kb + 4 * rr;
      const bool hv = h < hcnt;
      float x[U];
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = hv && (pb + u * step + kt < hi);
        x[u] = ok ? c4[u][rr] * ksc[u] : -INFINITY;
        mx = fmaxf(mx, x[u]);
      }
      const float mn = fmaxf(m_run[rr], row16_max(mx));
      const float mu = (mn == -INFINITY) ? 0.0f : mn;
      alpha[rr] = fast_exp2((m_run[rr] - mu) * p.c);
      float psum = 0.0f, csum = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float pw = fast_exp2((x[u] - mu) * p.c);
        const float wv = pw * vsc[u];
        psum += pw;
        csum += wv;
        if (h < HG) s_w[w][u][kt][h] = wv;
      }
      l_run[rr] = l_run[rr] * alpha[rr] + psum;
      if constexpr (F::QUANT) c_run[rr] = c_run[rr] * alpha[rr] + csum;
      m_run[rr] = mn;
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
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < F::VLD; ++j) {
        const int tl = j * F::TPL + vt;
        float wt[HG];
#pragma unroll
        for (int h = 0; h < HG; ++h) wt[h] = s_w[w][u][tl][h];
        float f[F::EV];
        F::vconv(vr[u][j], f);
#pragma unroll
        for (int h = 0; h < HG; ++h)
#pragma unroll
          for (int e = 0; e < F::EV; ++e) acc[h][e] = fmaf(wt[h], f[e], acc[h][e]);
      }
    }
    compiler_fence();
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
    for (int e = 0; e < F::EV; ++e) acc[h][e] = sum_over_token_rows<F::LPR>(acc[h][e]);
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
        s_m[h][w] = m_run[rr];
        s_l[h][w] = l_run[rr];
      }
    }
  }
  __syncthreads();

  // ---- merge the waves, emit output or split scratch ----
  // Each (head, d) thread forms the waves' weights e^(m_w - M) itself from
  // the head's LDS row (an empty wave, m = -inf, weighs 0; an empty split
  // keeps M = -inf).
  for (int idx = threadIdx.x; idx < hcnt * D; idx += blockDim.x) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = -INFINITY;
    for (int ww = 0; ww < nw; ++ww) M = fmaxf(M, s_m[h][ww]);
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
      for (int ww = 0; ww < nw; ++ww) {
        const float sc = fast_exp2((s_m[h][ww] - M) * p.c);
        L += sc * s_l[h][ww];
        O += sc * s_o[ww][h][d];
      }
    }
    const size_t qh = qrow0 + h;
    if (p.direct) {
      p.o[qh * D + d] = (_Float16)(O / L);
    } else {
      const size_t b = qh * p.S + s;
      const float mo = (M == -INFINITY) ? -INFINITY : M * p.scale;
      if (p.slot >= 0) {  // device-scope stores: read by another workgroup of this launch
        if (d == 0) {
          __hip_atomic_store(p.m_part + b, mo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(p.l_part + b, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __hip_atomic_store(p.o_part + b * D + d, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (d == 0) {
          p.m_part[b] = mo;
          p.l_part[b] = L;
        }
        p.o_part[b * D + d] = O;
      }
    }
  }

  // ---- in-kernel split merge: the last of the S workgroups of this
  // (KV row, head group) merges the S partials of its heads. The partials
  // above were stored at device scope (sc1, past the non-coherent per-XCD
  // L2s); each thread waits for its stores to complete before the barrier,
  // so by the time thread 0 counts the workgroup in, its partials are
  // visible device-wide. The last arriver reads every partial with
  // device-scope loads. No L2 writeback or invalidate is needed, and nobody
  // waits on the counter, so no workgroup can stall.
  if (!p.direct && p.slot >= 0) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      int* ctr = &g_split_arrivals[p.slot][blockIdx.x / p.S];
      const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == p.S - 1;
      if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (s_last) merge_splits<D, true>(p.m_part, p.l_part, p.o_part, p.o, qrow0, hcnt, p.S, s_macc, s_mred);
  }
}

// Two-kernel form of the split merge (decode_attn_gqa_sk_fast.cu:57-94): one
// workgroup per query head. Used when a call cannot take arrival counters.
template <int D>
__global__ void __launch_bounds__(64 * NW_MAX) combine_kernel(const float* __restrict__ m_part,
                                                              const float* __restrict__ l_part,
                                                              const float* __restrict__ o_part,
                                                              _Float16* __restrict__ o, int S) {
  __shared__ fl4_t s_acc[64 * NW_MAX];
  __shared__ float s_red[2 * 64 * NW_MAX / (D / 4)];
  merge_splits<D, false>(m_part, l_part, o_part, o, blockIdx.x, 1, S, s_acc, s_red);
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
