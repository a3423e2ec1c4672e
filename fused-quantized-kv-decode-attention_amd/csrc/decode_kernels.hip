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
//   1. has loaded the K tile as matrix-core operand A (int8 / int4: lane l
//      token l % 16, 64 contiguous bytes of 16 rows per dwordx4 instruction;
//      fp16: whole rows, rearranged through the wave's LDS rows) and the V
//      tile as four loads of 4 whole rows each,
//   2. computes the transposed scores S^T = K Q^T (tokens on M, query heads
//      on N) with D/32 v_mfma_f32_16x16x32_f16; column n carries head
//      n % HG, and lane l keeps the scores of tile (l % 16) / HG of each
//      group of 16 / HG tiles (column packing), tokens 4 (l / 16) .. + 3,
//   3. runs one online-softmax step per pass with v_exp_f32 (exp(x) =
//      2^(x log2 e), log2 e folded into the score scale) and an all-reduce
//      over the head's columns and the four lane rows; the weights p (times
//      the per-token V scale for int8/int4), as fp16 pairs hi + lo, are then
//      already in operand-B layout of
//   4. O^T += V^T P^T with D/16 v_mfma_f32_16x16x32_f16 per pair of tiles,
//      with four tokens of one head-dim element in each operand slot: fp16 /
//      bf16 lanes load their own four tokens' row segments; narrower rows
//      load four consecutive rows per instruction and a 4 x 4 exchange of
//      the V chunks between lane rows and registers (v_permlane32_swap /
//      v_permlane16_swap) regroups them (int8 / fp8 waves of one pass instead
//      score each group of four tokens in transposed order, so the tokens a
//      lane row scores are the ones whose V it loaded, and skip the exchange);
//      int8/int4 become exact fp16 on the
//      way. Each tile's weights enter operand B in the columns
//      0 .. HG-1 that are emitted (fp16: moved there by a DPP row shift) or
//      in the tile's own columns, the rest zero, summed at the end (int8 /
//      int4, whose products carry a bias until then).
// Waves of a workgroup take interleaved tiles; their (m, l, acc) states are
// merged through LDS. With one split the workgroup writes the normalised
// fp16 output; otherwise it writes the reference's fp32 scratch layout
// (m_part[h*S+s], l_part[h*S+s], o_part[(h*S+s)*D+d]), and the last of the
// S workgroups of its (KV row, head group) to finish merges the splits in
// the same launch (or, without an arrival-counter slot, the combine kernel
// does in a second launch).
//
// Two formats beyond the reference's ride the same code: bf16 rows move like
// fp16 and take the bf16 matrix-core product (the query and the weights as
// bf16 pairs: the query exact, the weights to 2^-16), and fp8 e4m3 codes move
// like int8 and convert to exact fp16 in hardware (no bias: per-token scales
// only).
//
// Reference algorithm: decode_attn_gqa_sk_fast.cu:6-54 (partial),
// :57-94 (combine); decode_attn_fp16_mw.cu:6-49 and decode_attn_gqa.cu:8-55
// are the single-split case; decode_attn_int8_mw.cu:6-51 and
// decode_attn_int4.cu:8-46 add per-token scales.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>
#include <numeric>

#include "kv_formats.h"
#include "launch.h"

namespace fqkv {

constexpr float LOG2E = 1.4426950408889634f;

// Timeline instrumentation, compiled in only with -DFQKV_TIMELINE: lane 0 of
// each wave records the 100 MHz real-time counter at the kernel's stages into
// g_timeline[workgroup][wave][stage], which fqkv_timeline_read copies to the
// host (or, with bytes = SIZE_MAX, clears).
#ifdef FQKV_TIMELINE
constexpr int TIMELINE_BLOCKS = 4096;
__device__ unsigned long long g_timeline[TIMELINE_BLOCKS][NW_MAX][16];
// The stamp takes its own copy of the workgroup id (an asm move the compiler
// cannot merge with the kernel's uses): indexing g_timeline with blockIdx.x
// itself under the lane-0 branch made the compiler carry the id in a vector
// register through the branch and reuse that copy in the kernel's index
// math, so every buffer descriptor built from it became per-lane and each
// buffer load a readfirstlane loop over the wave.
#define FQKV_STAMP(stage)                                                                          \
  do {                                                                                             \
    uint32_t blk_;                                                                                 \
    asm volatile("s_mov_b32 %0, %1" : "=s"(blk_) : "s"(blockIdx.x));                              \
    const unsigned long long t_ = __builtin_amdgcn_s_memrealtime();                                \
    if ((threadIdx.x & 63) == 0 && blk_ < TIMELINE_BLOCKS) g_timeline[blk_][threadIdx.x >> 6][stage] = t_; \
  } while (0)
extern "C" int fqkv_timeline_read(void* host, size_t bytes) {
  if (bytes == (size_t)-1) {
    static unsigned long long z[TIMELINE_BLOCKS][NW_MAX][16];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_timeline), z, sizeof(z));
  }
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_timeline), bytes);
}
#else
#define FQKV_STAMP(stage) \
  do {                    \
  } while (0)
#endif

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Row exchanges between the four 16-lane rows of a wave (all VALU):
// v_permlane32_swap trades rows 2,3 of its first operand for rows 0,1 of its
// second; v_permlane16_swap trades the odd rows of its first operand for the
// even rows of its second. The builtins return {first, second} after the
// trade (copied to scalars: this compiler's __builtin_bit_cast of a
// vector-element expression reads element 0 whatever the index).
__device__ __forceinline__ void swap_rows32(uint32_t& a, uint32_t& b) {
  const auto t = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  const uint32_t x = t[0], y = t[1];
  a = x;
  b = y;
}
__device__ __forceinline__ void swap_rows16(uint32_t& a, uint32_t& b) {
  const auto t = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  const uint32_t x = t[0], y = t[1];
  a = x;
  b = y;
}
// 4 x 4 exchange between lane rows and registers: afterwards row R of
// register j holds what row j of register R held.
__device__ __forceinline__ void exchange_4x4(uint32_t& a0, uint32_t& a1, uint32_t& a2, uint32_t& a3) {
  swap_rows32(a0, a2);
  swap_rows32(a1, a3);
  swap_rows16(a0, a1);
  swap_rows16(a2, a3);
}
// Maxima run on order-preserving integer keys of the fp32 bit patterns: a
// negative value has its magnitude bits flipped, so signed integer order is
// float order (-0 < +0; the map is its own inverse). fmaxf of a value that
// arrives through a lane move compiles to two canonicalising moves and the
// maximum; v_max_i32 needs neither and takes a DPP operand directly.
__device__ __forceinline__ int fkey(float x) {
  const int b = __builtin_bit_cast(int, x);
  return b ^ ((b >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float unkey(int k) { return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7FFFFFFF)); }
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_mov_dpp(x, CTRL, 0xF, 0xF, true);
}

// All-reduce over the four lane rows (lanes with equal lane % 16). Combining
// both outputs of each swap makes the result independent of which operand
// receives which rows.
__device__ __forceinline__ int rows4_max_key(int k) {
  uint32_t a = (uint32_t)k, b = a;
  swap_rows32(a, b);
  k = max((int)a, (int)b);
  a = (uint32_t)k;
  b = a;
  swap_rows16(a, b);
  return max((int)a, (int)b);
}
__device__ __forceinline__ float rows4_max(float x) { return unkey(rows4_max_key(fkey(x))); }
__device__ __forceinline__ float rows4_sum(float x) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  swap_rows32(a, b);
  x = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  a = __builtin_bit_cast(uint32_t, x);
  b = a;
  swap_rows16(a, b);
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

typedef float fl4_t __attribute__((ext_vector_type(4)));

// Arrival counters of the in-kernel split merge. Zero at load; the workgroup
// that merges a group resets its counter, so every call leaves them at zero.
// Device-scope atomics on one cache line serialise, so the counters of
// consecutive groups sit 256 bytes apart (group g of a slot at int
// (g % 256) * 64 + g / 256): with them packed, every workgroup of a call
// queued on the same one or two lines, and the merge's cost moved with the
// array's alignment. 256-byte alignment keeps the lines of different groups
// apart.
constexpr int ARRIVAL_LINES = 256;
static_assert(MAX_SPLIT_GROUPS % ARRIVAL_LINES == 0 && MAX_SPLIT_GROUPS / ARRIVAL_LINES <= 64,
              "arrival counters: at most 64 per 256-byte line");
__device__ __attribute__((aligned(256))) int g_split_arrivals[SPLIT_SLOTS][MAX_SPLIT_GROUPS];
__device__ __forceinline__ int* arrival_counter(int slot, uint32_t group) {
  return &g_split_arrivals[slot][(group % ARRIVAL_LINES) * 64 + group / ARRIVAL_LINES];
}

// Full-wave reductions: DPP within each 16-lane row (quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror), then across the rows.
// Every pattern used here reads a lane of the same row, so bound_ctrl (zero
// for a source outside the row) never applies; setting it lets the compiler
// fold the move into the consuming add (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float wave_max(float x) {
  int k = fkey(x);
  k = max(k, dpp_i<0xB1>(k));
  k = max(k, dpp_i<0x4E>(k));
  k = max(k, dpp_i<0x141>(k));
  k = max(k, dpp_i<0x140>(k));
  return unkey(rows4_max_key(k));
}
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f<0xB1>(x);
  x += dpp_f<0x4E>(x);
  x += dpp_f<0x141>(x);
  x += dpp_f<0x140>(x);
  return rows4_sum(x);
}

// Column packing of the score product. A 16 x 16 score tile has 16 head
// columns but a work item has only HG query heads, so P = min(U, 16 / HG)
// tiles of a pass share one column set: column n holds head n % HG of tile
// n / HG of each group of P tiles. cols_fold combines the P columns of each
// head within a 16-lane row (DPP quad_perm xor 1 / xor 2, row_ror 4 / 8);
// columns past P * HG take part in HG = 2 and in HG = 1 with P = 8 (whose
// fold covers the whole row) and must hold a neutral value (or, for a
// maximum, any value of the same pass).
// (Sums on fp32 values, maxima on integer keys.)
template <int HG, int P, typename T, typename Op, typename Mv>
__device__ __forceinline__ T cols_fold(T x, Op op, Mv mv) {
  if constexpr (P == 1) {
    return x;
  } else if constexpr (HG == 1 && P <= 4) {  // columns 0..3: one quad
    x = op(x, mv(x, std::integral_constant<int, 0xB1>()));
    return op(x, mv(x, std::integral_constant<int, 0x4E>()));
  } else if constexpr (HG == 1) {  // columns 0..P-1: the whole row
    x = op(x, mv(x, std::integral_constant<int, 0xB1>()));
    x = op(x, mv(x, std::integral_constant<int, 0x4E>()));
    x = op(x, mv(x, std::integral_constant<int, 0x124>()));
    return op(x, mv(x, std::integral_constant<int, 0x128>()));
  } else if constexpr (HG == 2) {  // columns hh, hh + 2, hh + 4, hh + 6
    x = op(x, mv(x, std::integral_constant<int, 0x4E>()));
    x = op(x, mv(x, std::integral_constant<int, 0x124>()));
    return op(x, mv(x, std::integral_constant<int, 0x128>()));
  } else if constexpr (HG == 4) {  // columns hh + 4 j, j = 0..3
    x = op(x, mv(x, std::integral_constant<int, 0x124>()));
    return op(x, mv(x, std::integral_constant<int, 0x128>()));
  } else {  // HG == 8, P == 2: columns hh, hh + 8
    static_assert(HG == 8 && P == 2, "column packing");
    return op(x, mv(x, std::integral_constant<int, 0x128>()));
  }
}
template <int HG, int P>
__device__ __forceinline__ float cols_sum(float x) {
  return cols_fold<HG, P>(
      x, [](float a, float b) { return a + b; }, [](float v, auto c) { return dpp_f<decltype(c)::value>(v); });
}
template <int HG, int P>
__device__ __forceinline__ int cols_max_key(int k) {
  return cols_fold<HG, P>(
      k, [](int a, int b) { return max(a, b); }, [](int v, auto c) { return dpp_i<decltype(c)::value>(v); });
}
// Maximum of a head over its P columns and the four lane rows (NONNEG: the
// values are >= 0, whose bit patterns are their own keys).
template <int HG, int P, bool NONNEG = false>
__device__ __forceinline__ float head_max(float x) {
  if constexpr (NONNEG)
    return __builtin_bit_cast(float, rows4_max_key(cols_max_key<HG, P>(__builtin_bit_cast(int, x))));
  else
    return unkey(rows4_max_key(cols_max_key<HG, P>(fkey(x))));
}

// f(jl) for the lane's tile index jl < P. The selects are bitwise blends
// under the loop-invariant lane masks m[i] = -((jl >> i) & 1) (one bitwise
// select each, P - 1 per pick): written as conditionals, the compiler turns
// the chain into a per-lane indexed array in scratch memory.
template <typename T>
__device__ __forceinline__ T blend(uint32_t m, T a, T b) {  // m ? b : a
  static_assert(sizeof(T) == 4, "32-bit values");
  const uint32_t x = __builtin_bit_cast(uint32_t, a), y = __builtin_bit_cast(uint32_t, b);
  return __builtin_bit_cast(T, (x & ~m) | (y & m));
}
// Lane n of each 16-lane row takes lane n + sh of the row (0 past its end):
// DPP row_shl, sh a compile-time constant once the caller's loop is unrolled.
template <int SH>
__device__ __forceinline__ uint32_t row_shl_c(uint32_t x) {
  if constexpr (SH == 0)
    return x;
  else
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x100 + SH, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t row_shl(uint32_t x, int sh) {
  switch (sh) {
    case 1: return row_shl_c<1>(x);
    case 2: return row_shl_c<2>(x);
    case 3: return row_shl_c<3>(x);
    case 4: return row_shl_c<4>(x);
    case 5: return row_shl_c<5>(x);
    case 6: return row_shl_c<6>(x);
    case 7: return row_shl_c<7>(x);
    case 8: return row_shl_c<8>(x);
    case 9: return row_shl_c<9>(x);
    case 10: return row_shl_c<10>(x);
    case 11: return row_shl_c<11>(x);
    case 12: return row_shl_c<12>(x);
    case 13: return row_shl_c<13>(x);
    case 14: return row_shl_c<14>(x);
    case 15: return row_shl_c<15>(x);
    default: return x;
  }
}

template <int P, int J0 = 0, typename Fn>
__device__ __forceinline__ auto pick(const uint32_t (&m)[4], Fn f) {
  static_assert(P == 1 || P == 2 || P == 4 || P == 8 || P == 16, "column packing");
  if constexpr (P == 1) {
    return f(J0);
  } else {
    constexpr int B = P == 2 ? 0 : (P == 4 ? 1 : (P == 8 ? 2 : 3));  // the bit that halves [J0, J0 + P)
    return blend(m[B], pick<P / 2, J0>(m, f), pick<P / 2, J0 + P / 2>(m, f));
  }
}

// Merge S split partials for query heads h0 .. h0+nh-1:
// o[h] = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s
// (decode_attn_gqa_sk_fast.cu:57-94; m in natural-log units, an empty split
// has m = -inf, l = 0, acc = 0 and weight 0; an empty sequence, where every
// split is empty, gives zeros).
//
// A unit is one head's 64-dim block; one wave merges one unit. Lane s forms
// the weight of split s of each 64-split block (kept in the wave's own LDS
// row, so no barrier is needed to share it); the partials arrive as 16-byte
// loads, lane (k, q) = (lane / 16, lane % 16) reading dims 4q .. 4q+3 of
// split 4j + k with load j, so a chunk of 32 splits is 8 loads per lane. A
// CU issues a vector memory instruction every ~16 cycles whatever its width,
// so 4-byte loads (one dim per lane) made the merge's loads, not its
// latency, the cost: 34 of them per wave took ~1.8 us per merge on MI355X.
// The four lane rows' sums are then added across rows. Buffer descriptors
// end at the last split (the whole byte offset is the VGPR offset, which the
// raw-buffer range check covers), so loads past it return zero and no lane
// tests bounds per load. The m and l loads go out with the first chunk, so a
// merge of up to 32 splits is one memory round trip. When there are fewer
// units than waves, the splits of a unit are cut into nsl slices on different
// waves that meet in LDS (the merge's only barrier; its condition is the same
// for the whole workgroup). With at most CHK splits and no more units than
// waves everything is one chunk per wave, and a short path skips the slice
// bookkeeping.
// CPOL: cache policy of the partial loads (CPOL_SC1 for partials that other
// workgroups of the same launch stored at device scope).
// s_w: 64 floats per wave (16-byte aligned rows); s_red: 65 floats per wave.
template <int D, int CPOL>
__device__ __forceinline__ void merge_splits(const float* __restrict__ m_part, const float* __restrict__ l_part,
                                             const float* __restrict__ o_part, _Float16* __restrict__ o,
                                             size_t h0, int nh, int S, float (*s_w)[64], float (*s_red)[65]) {
  constexpr int DB = D / 64;  // units per head
  constexpr int CHK = 32;     // splits per chunk: 8 loads of 4 splits per lane
  constexpr int NJ = CHK / 4;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int units = nh * DB;
  const int kr = lane >> 4;                          // split within a load: 4 j + kr
  const uint32_t qo = 16u * (uint32_t)(lane & 15);   // byte offset of dims 4q .. 4q+3 in the unit
  auto ld = [](rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, CPOL));
  };
  auto ld4 = [](rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(fl4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CPOL));
  };
  // after the row sums every lane row holds the unit's 64 sums; lane (k, q)
  // writes dim 4q + k, so one 2-byte store per lane covers the unit
  auto put = [&](_Float16* unit, int i, float v, float L) {  // output dim i of a 64-dim unit
    unit[i] = L > 0.0f ? (_Float16)(v / L) : (_Float16)0.0f;
  };
  auto emit = [&](fl4_t a, float L, _Float16* dst) {
    // lane row kr needs component kr summed over the four lane rows: after a
    // 4 x 4 exchange, register j of row kr holds component kr of row j
    // (components copied to scalars first: a bit cast of a vector-element
    // expression reads element 0 with this compiler, whatever the index)
    const float ax = a.x, ay = a.y, az = a.z, aw = a.w;
    uint32_t a0 = __builtin_bit_cast(uint32_t, ax), a1 = __builtin_bit_cast(uint32_t, ay),
             a2 = __builtin_bit_cast(uint32_t, az), a3 = __builtin_bit_cast(uint32_t, aw);
    exchange_4x4(a0, a1, a2, a3);
    const float v = (__builtin_bit_cast(float, a0) + __builtin_bit_cast(float, a2)) +
                    (__builtin_bit_cast(float, a1) + __builtin_bit_cast(float, a3));
    put(dst, 4 * (lane & 15) + kr, v, L);
  };
  if (S <= CHK && units <= nw) {
    // One chunk per unit and a wave per unit (the batch-1 split-K case):
    // wave wv merges unit wv with no slice bookkeeping, so its loads leave
    // a few scalar instructions after the merge is known to be needed.
    if (wv < units) {
      const int h = wv / DB;
      const size_t hrow = h0 + h;
      const rsrc_t rM = make_rsrc(m_part + hrow * S, (uint32_t)S * 4u);
      const rsrc_t rL = make_rsrc(l_part + hrow * S, (uint32_t)S * 4u);
      const rsrc_t rO = make_rsrc(o_part + hrow * S * D + (wv - h * DB) * 64, (uint32_t)(S - 1) * D * 4u + 256u);
      const float m0 = ld(rM, 4u * (uint32_t)lane);
      const float l0 = ld(rL, 4u * (uint32_t)lane);
      fl4_t ov[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) ov[j] = ld4(rO, (uint32_t)((4 * j + kr) * D * 4) + qo);  // zero past split S - 1
      float M = wave_max(lane < S ? m0 : -INFINITY);
      FQKV_STAMP(8);  // merge: maximum over the splits known
      if (M == -INFINITY) M = 0.0f;  // every split empty: all weights 0
      const float w = lane < S ? fast_exp2((m0 - M) * LOG2E) : 0.0f;
      s_w[wv][lane] = w;
      const float L = wave_sum(w * l0);
      fl4_t acc4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float wk = s_w[wv][4 * j + kr];
        acc4.x = fmaf(wk, ov[j].x, acc4.x);
        acc4.y = fmaf(wk, ov[j].y, acc4.y);
        acc4.z = fmaf(wk, ov[j].z, acc4.z);
        acc4.w = fmaf(wk, ov[j].w, acc4.w);
      }
      emit(acc4, L, o + hrow * D + (wv - h * DB) * 64);
    }
    return;
  }
  // nsl = 2^lg slices per unit; waves wv with equal wv >> lg share a unit
  int lg = 0;
  while ((2 << lg) * units <= nw && (2 << lg) * CHK <= S) ++lg;
  const int nsl = 1 << lg;
  const int cu = nw >> lg;                                              // units per round
  const int len = (((S + nsl - 1) >> lg) + CHK - 1) & ~(CHK - 1);      // splits per slice
  for (int ub = 0; ub < units; ub += cu) {  // a single round when nsl > 1
    const int u = ub + (wv >> lg);
    const int sl = wv & (nsl - 1);
    const int h = u / DB;
    const int db = u - h * DB;
    const int start = sl * len;
    const int end = min(S, start + len);
    const bool live = (wv >> lg) < cu && u < units && start < end;  // wave-uniform
    fl4_t acc4 = {0.0f, 0.0f, 0.0f, 0.0f};
    float L = 0.0f;
    if (live) {
      const size_t hrow = h0 + h;
      const rsrc_t rM = make_rsrc(m_part + hrow * S, (uint32_t)S * 4u);
      const rsrc_t rL = make_rsrc(l_part + hrow * S, (uint32_t)S * 4u);
      // split start + i, dims 4q .. 4q+3 at byte i D 4 + qo; the record ends
      // with the slice's last split's 64 dims
      const rsrc_t rO = make_rsrc(o_part + (hrow * S + start) * D + db * 64,
                                  (uint32_t)(end - start - 1) * D * 4u + 256u);
      const uint32_t lo4 = (uint32_t)lane * 4u;
      const float m0 = ld(rM, lo4);
      const float l0 = ld(rL, lo4);
      fl4_t ov[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) ov[j] = ld4(rO, (uint32_t)((4 * j + kr) * D * 4) + qo);
      float M = lane < S ? m0 : -INFINITY;
      for (int s0 = 64; s0 < S; s0 += 64) {
        const float mm = ld(rM, lo4 + (uint32_t)s0 * 4u);
        M = fmaxf(M, s0 + lane < S ? mm : -INFINITY);
      }
      M = wave_max(M);
      if (M == -INFINITY) M = 0.0f;  // every split empty: all weights 0
      for (int c0 = start; c0 < end; c0 += CHK) {
        const int b = c0 >> 6;
        if (c0 == start || (c0 & 63) == 0) {  // weights of splits 64 b .. 64 b + 63 in this slice
          float mm = m0, ll = l0;
          if (b > 0) {
            mm = ld(rM, lo4 + (uint32_t)b * 256u);
            ll = ld(rL, lo4 + (uint32_t)b * 256u);
          }
          const int sk = 64 * b + lane;
          const float w = sk >= start && sk < end ? fast_exp2((mm - M) * LOG2E) : 0.0f;
          L = fmaf(w, ll, L);
          s_w[wv][lane] = w;
        }
        auto accumulate = [&](const fl4_t (&v)[NJ]) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const float wk = s_w[wv][(c0 & 63) + 4 * j + kr];
            acc4.x = fmaf(wk, v[j].x, acc4.x);
            acc4.y = fmaf(wk, v[j].y, acc4.y);
            acc4.z = fmaf(wk, v[j].z, acc4.z);
            acc4.w = fmaf(wk, v[j].w, acc4.w);
          }
        };
        const int c1 = c0 + CHK;
        if (c1 < end) {
          fl4_t nv[NJ];
#pragma unroll
          for (int j = 0; j < NJ; ++j) nv[j] = ld4(rO, (uint32_t)((c1 - start + 4 * j + kr) * D * 4) + qo);
          accumulate(ov);
#pragma unroll
          for (int j = 0; j < NJ; ++j) ov[j] = nv[j];
        } else {
          accumulate(ov);
        }
      }
      L = wave_sum(L);
    }
    if (nsl > 1) {
      // slices meet in LDS: the row sums first, then lane (k, q) parks dim 4q + k
      if (live) {
        acc4.x = rows4_sum(acc4.x);
        acc4.y = rows4_sum(acc4.y);
        acc4.z = rows4_sum(acc4.z);
        acc4.w = rows4_sum(acc4.w);
        s_red[wv][4 * (lane & 15) + kr] = kr == 0 ? acc4.x : (kr == 1 ? acc4.y : (kr == 2 ? acc4.z : acc4.w));
        if (lane == 0) s_red[wv][64] = L;
      }
      __syncthreads();
      if (live && sl == 0) {
        float a = s_red[wv][lane];
        for (int q = 1; q < nsl; ++q) {
          if ((q * len) >= S) break;  // empty slice
          a += s_red[wv + q][lane];
          L += s_red[wv + q][64];
        }
        put(o + (h0 + h) * D + db * 64, lane, a, L);
      }
    } else if (live) {
      emit(acc4, L, o + (h0 + h) * D + db * 64);
    }
  }
}

// Row pitch of the per-wave accumulator rows in LDS: 4 floats of padding
// spread the wave's float4 writes over more banks.
template <int D>
constexpr int opitch() { return D + 4; }

// Merge the NWC waves' (m, l, acc) of a workgroup through LDS and emit the
// normalised fp16 output (one split) or the split's fp32 partials. Thread t
// takes four consecutive elements 4t .. 4t+3 of the workgroup's hcnt x D
// outputs (head h = 4t / D): one pass whenever HG x D <= 256 x waves (every
// shape here with 4 or 8 waves; 4 heads of 128 with 2 waves, the one-token
// split, took four passes at one element per thread, 1.6 us of a 5 us
// call). Each thread forms its head's wave weights
// e^(m_w - M) itself from the head's LDS rows (read whole; every lane of a head
// reads the same address), adds the NWC waves' float4 of acc, and stores 16
// bytes of partials or four fp16 outputs. An empty wave (m = -inf) weighs 0
// and an empty split keeps M = -inf with l = acc = 0. The l sum is the
// pairwise tree (w0 l0 + w1 l1) + (w2 l2 + w3 l3) + ..., the acc sum goes
// wave by wave.
template <int N>
__device__ __forceinline__ void lds_row(const float* src, float (&v)[N]) {
  if constexpr (N == 2) {
    const float2 a = *reinterpret_cast<const float2*>(src);
    v[0] = a.x;
    v[1] = a.y;
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const fl4_t a = *reinterpret_cast<const fl4_t*>(src + i);
      v[i] = a.x;
      v[i + 1] = a.y;
      v[i + 2] = a.z;
      v[i + 3] = a.w;
    }
  }
}
template <int N>
__device__ __forceinline__ float tree_sum(const float (&v)[N]) {
  if constexpr (N == 2) {
    return v[0] + v[1];
  } else if constexpr (N == 4) {
    return (v[0] + v[1]) + (v[2] + v[3]);
  } else {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  }
}

template <int D, int HG, int NWC>
__device__ __forceinline__ void merge_waves_emit(const PartialParams& p, const float (*s_o)[HG][opitch<D>()],
                                                 const float (*s_m)[NW_MAX], const float (*s_l)[NW_MAX],
                                                 size_t qrow0, int hcnt, int s) {
  static_assert(NWC == 2 || NWC == 4 || NWC == 8, "waves per workgroup");
  for (int idx = 4 * (int)threadIdx.x; idx < hcnt * D; idx += 4 * (int)blockDim.x) {
    const int h = idx / D;
    const int d = idx - h * D;
    float mw[NWC], lw[NWC];
    fl4_t a[NWC];
    lds_row<NWC>(s_m[h], mw);
    lds_row<NWC>(s_l[h], lw);
#pragma unroll
    for (int ww = 0; ww < NWC; ++ww) a[ww] = *reinterpret_cast<const fl4_t*>(&s_o[ww][h][d]);
    // every LDS read of the merge in flight before the first use: left to
    // itself the compiler issued the waves' acc rows one or two at a time,
    // behind the maximum and the weights, a chain of LDS round trips
    __builtin_amdgcn_sched_barrier(0);
    float M = mw[0];
#pragma unroll
    for (int j = 1; j < NWC; ++j) M = fmaxf(M, mw[j]);
    const float Mu = (M == -INFINITY) ? 0.0f : M;
    float wj[NWC], wl[NWC];
#pragma unroll
    for (int j = 0; j < NWC; ++j) {
      wj[j] = fast_exp2((mw[j] - Mu) * p.c);
      wl[j] = wj[j] * lw[j];
    }
    const float L = tree_sum<NWC>(wl);
    fl4_t O = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ww = 0; ww < NWC; ++ww) {
      O.x = fmaf(wj[ww], a[ww].x, O.x);
      O.y = fmaf(wj[ww], a[ww].y, O.y);
      O.z = fmaf(wj[ww], a[ww].z, O.z);
      O.w = fmaf(wj[ww], a[ww].w, O.w);
    }
    const size_t qh = qrow0 + h;
    // normalised fp16 output (an empty sequence gives zeros)
    auto put_out = [&]() {
      _Float16* dst = p.o + qh * D + d;
      const float Ox = O.x, Oy = O.y, Oz = O.z, Ow = O.w;
      dst[0] = L > 0.0f ? (_Float16)(Ox / L) : (_Float16)0.0f;
      dst[1] = L > 0.0f ? (_Float16)(Oy / L) : (_Float16)0.0f;
      dst[2] = L > 0.0f ? (_Float16)(Oz / L) : (_Float16)0.0f;
      dst[3] = L > 0.0f ? (_Float16)(Ow / L) : (_Float16)0.0f;
    };
    if (p.direct) {
      put_out();
    } else {
      const size_t b = qh * p.S + s;
      float* orow = p.o_part + b * D + d;
      const float mo = (M == -INFINITY) ? -INFINITY : M * p.scale;
      if (p.slot >= 0) {
        // 16-byte stores of the lane's four partials through a descriptor
        // from the wave's first head row (a wave spans at most 64 / (D / 4)
        // heads; rows of consecutive heads lie S x D floats apart)
        const int h0 = __builtin_amdgcn_readfirstlane(h);
        const rsrc_t rP = make_rsrc(p.o_part + ((qrow0 + h0) * p.S + s) * D,
                                    ((uint32_t)(64 * 4 / D - 1) * (uint32_t)p.S * D + D) * 4u);
        const int off = ((h - h0) * p.S * D + d) * 4;
        const u4_t bits = __builtin_bit_cast(u4_t, O);
        if (p.xcd_local) {  // read by a workgroup on this XCD: its L2 is the meeting point
          if (d == 0) {
            __hip_atomic_store(p.m_part + b, mo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_store(p.l_part + b, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          }
          __builtin_amdgcn_raw_buffer_store_b128(bits, rP, off, 0, CPOL_SC0);
        } else {  // device-scope stores: read by another workgroup of this launch
          if (d == 0) {
            __hip_atomic_store(p.m_part + b, mo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.l_part + b, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          __builtin_amdgcn_raw_buffer_store_b128(bits, rP, off, 0, CPOL_SC1);
        }
      } else {
        if (d == 0) {
          p.m_part[b] = mo;
          p.l_part[b] = L;
        }
        *reinterpret_cast<fl4_t*>(orow) = O;  // o_part is 16-byte aligned and D a multiple of 4
      }
      // one split: the workgroup holds the whole result, so it writes the
      // output too and no merge follows (one launch per call)
      if (p.S == 1) put_out();
    }
  }
}

// Forces the launch constants into scalar registers at this point (an empty
// asm that reads them), so the compiler issues their kernel-argument loads as
// one batch instead of next to each first use.
template <typename T>
__device__ __forceinline__ void pin_s(T v) {
  asm volatile("" ::"s"(v));
}
template <bool QUANT, bool PAGED>
__device__ __forceinline__ void pin_sgprs(const PartialParams& p) {
  pin_s(p.q); pin_s(p.K); pin_s(p.V);
  pin_s(p.G); pin_s(p.N); pin_s(p.chunk); pin_s(p.ngroups); pin_s(p.c);
  pin_s(p.hkv); pin_s(p.kv_hs); pin_s(p.kv_ts);
  pin_s(p.split_major); pin_s(p.blk_d);
  pin_s(p.div_blk.magic); pin_s(p.div_blk.shift); pin_s(p.div_groups.magic); pin_s(p.div_groups.shift);
  pin_s(p.div_hkv.magic); pin_s(p.div_hkv.shift); pin_s(p.hg_k); pin_s(p.hg_d);
  if constexpr (!PAGED) pin_s(p.kv_bs);
  if constexpr (QUANT) {
    pin_s(p.Ks); pin_s(p.Vs); pin_s(p.sc_hs); pin_s(p.sc_ts);
    if constexpr (!PAGED) pin_s(p.sc_bs);
  }
  if constexpr (PAGED) {
    pin_s(p.kv_bs); pin_s(p.page_table); pin_s(p.seq_lens); pin_s(p.max_pages); pin_s(p.page_log2);
    pin_s(p.num_pages);
    if constexpr (QUANT) pin_s(p.sc_bs);
  }
}

// PVV: P.V on the vector ALUs instead of the matrix cores (fp16, contiguous
// rows only): a measurement variant for comparing the two, selected by
// fqkv_set_pv_valu. Each wave writes its fp32 weights to its own LDS rows
// and every lane multiplies the V elements it holds after the row exchange
// (tokens 4R .. 4R+3, elements VE i .. VE i + VE-1 of each tile) by the
// weights of those tokens for each of its heads.
// 16-token tiles a wave loads per pass (one online-softmax step per pass).
// With one query head per work item, column packing gives each tile of the
// pass its own score column, so a pass of U tiles keeps U of the 16 columns
// busy and the softmax instructions of a pass are shared by U tiles. Eight
// tiles pay off for contiguous int4 at D 64, whose 32-byte rows leave the
// registers for them (124 VGPRs, 4 waves per SIMD): MHA B 2048, N 4096
// 100.6 -> 95.7 us, B 256 19.2 -> 17.4 us. Measured slower, and kept at four:
// int4 at D 128 (B 256 +14 %), int8 at D 64 (B 256 +12 %), sixteen tiles for
// int4 (B 2048 +8 % at D 64; 2 waves per SIMD), and the paged rows (2 waves).
// SHORT: two tiles (the fewest the paired P.V products take), for splits of
// at most two tiles per wave on contiguous rows, where a four-tile pass issues
// loads, address arithmetic and products for tiles past the split's end.
// Same-box A/B, split-K D 128, batch 1: fp16 at N 512 / 2048 / 4096 / 8192
// 5.55 -> 5.24, 6.81 -> 6.20, 8.31 -> 7.36, 10.01 -> 9.33 us; int8 6.62 ->
// 6.00, 7.14 -> 6.50, 8.56 -> 7.56, 9.02 -> 8.28 us; int4 6.30 -> 5.77,
// 6.57 -> 6.01, 7.65 -> 6.94, 7.85 -> 6.99 us; N 16384 (four tiles per wave,
// the usual pass) unchanged.
template <int FMT, int D, int HG, bool PAGED, bool PVV, bool SHORT = false>
constexpr int tiles_per_pass() {
  return SHORT ? 2 : ((FMT == KV_I4 && D == 64 && HG == 1 && !PAGED && !PVV) ? 8 : 4);
}

// KEEPV: int4 rows token-major without pages (heads sharing cache lines, the
// launcher's head grouping on), whose V loads go without the non-temporal hint.
// LAZY (int8 / int4 / fp8 / bf16, each wave one four-tile pass): the query's
// derived operands are formed, and a pass's scales unpacked, only once the
// pass's K and V loads are all out (see qprep and the scale loads below);
// with several passes per wave the registers this keeps live cost occupancy.
template <int FMT, int D, int HG, bool PAGED, bool PVV = false, bool KEEPV = false, bool SHORT = false,
          bool LAZY = false>
__global__ void __launch_bounds__(64 * NW_MAX) decode_partial_kernel(PartialParams p) {
  using F = Fmt<FMT, D>;
  static_assert(!PVV || (FMT == KV_F16 && !PAGED), "P.V on the vector ALUs: fp16, contiguous rows");
  using VG = VGeom<F::ROWB, D>;
  static_assert(!SHORT || (!PAGED && !PVV && !KEEPV), "short passes: contiguous rows");
  static_assert(!LAZY || (!PAGED && !PVV && !KEEPV), "lazy preparation: contiguous rows");
  constexpr int U = tiles_per_pass<FMT, D, HG, PAGED, PVV, SHORT>();
  constexpr int VE = VG::VE;   // PV steps per tile
  constexpr int VD = VG::VD;   // dwords per V chunk
  __shared__ __attribute__((aligned(16))) float s_o[NW_MAX][HG][opitch<D>()];
  __shared__ __attribute__((aligned(16))) float s_m[HG][NW_MAX];
  __shared__ __attribute__((aligned(16))) float s_l[HG][NW_MAX];
  __shared__ __attribute__((aligned(16))) float s_mw[NW_MAX][64];  // in-kernel split merge
  __shared__ float s_mr[NW_MAX][65];
  __shared__ int s_last;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_kstage[];  // fp16 K staging, F::KSTAGE bytes per wave

  FQKV_STAMP(0);  // start
  const int lane = threadIdx.x & 63;
  // wave index as a scalar, so tile loops branch per wave, not per lane
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  // blockIdx.x = s * nwsg + wsg or wsg * S + s (wsg = r * ngroups + hg),
  // decomposed with multiply-shift divisions
  // Every launch constant in one scalar-load round trip: read here, in the
  // entry block, so the loads leave together (lazily placed, they took four
  // dependent round trips before the first KV load, and one more before the
  // epilogue).
  pin_sgprs<F::QUANT, PAGED>(p);
  const uint32_t bq = fast_div(blockIdx.x, p.div_blk);
  const uint32_t br = blockIdx.x - bq * (uint32_t)p.blk_d;
  uint32_t wsg = p.split_major ? br : bq;
  const int s = (int)(p.split_major ? bq : br);
  {
    // in a block of 2^(hg_k + hg_d) groups, group e 2^hg_d + c becomes row c 2^hg_k + e:
    // head e of head set c, the set's heads 2^hg_d groups apart (the identity
    // when hg_k = hg_d = 0; no branch, so the prologue stays one block)
    const uint32_t k = (uint32_t)p.hg_k, d = (uint32_t)p.hg_d;
    const uint32_t low = wsg & ((1u << (k + d)) - 1u);
    wsg = (wsg - low) | ((low & ((1u << d) - 1u)) << k) | (low >> d);
  }
  const uint32_t rr = fast_div(wsg, p.div_groups);
  const int hg = (int)(wsg - rr * (uint32_t)p.ngroups);
  const int r = (int)rr;
  // KV row r = (sequence b, KV head h); its tokens sit kv_ts bytes apart
  const int b = (int)fast_div((uint32_t)r, p.div_hkv);
  const int h = r - b * p.hkv;
  const uint32_t ts = (uint32_t)p.kv_ts;
  int nr = p.N;  // tokens of this row
  if constexpr (PAGED) nr = min(min(p.seq_lens[b], p.N), p.max_pages << p.page_log2);
  const int lo = s * p.chunk;
  const int hi = min(lo + p.chunk, nr);
  const int hbase = hg * HG;
  const int hcnt = min(HG, p.G - hbase);
  const size_t qrow0 = (size_t)r * p.G + hbase;
  // base of the row's token 0 (paged: of the row's head within a page)
  const uint8_t* Kr = p.K + (PAGED ? 0 : (size_t)b * p.kv_bs) + (size_t)h * p.kv_hs;
  const uint8_t* Vr = p.V + (PAGED ? 0 : (size_t)b * p.kv_bs) + (size_t)h * p.kv_hs;
  const _Float16* Ksr = F::QUANT ? p.Ks + (PAGED ? 0 : (size_t)b * p.sc_bs) + (size_t)h * p.sc_hs : nullptr;
  const _Float16* Vsr = F::QUANT ? p.Vs + (PAGED ? 0 : (size_t)b * p.sc_bs) + (size_t)h * p.sc_hs : nullptr;

  const int n = lane & 15;  // column of S^T, P^T and O^T; token row of the K operand
  const int R = lane >> 4;  // lane row: K dword group; scores and V of tokens 4R .. 4R+3 (TPERM: R + 4k)
  // Column packing (cols_fold): column n carries head hh of tile jl of each
  // group of P tiles; columns past P * HG carry nothing (scores masked).
  constexpr int P = (16 / HG < U) ? 16 / HG : U;
  constexpr int NG = U / P;  // tile groups per pass
  const bool live = n < P * HG;
  const int jl = live ? n / HG : P - 1;
  const int hh = n % HG;
  const uint32_t jm[4] = {(jl & 1) ? ~0u : 0u, (jl & 2) ? ~0u : 0u, (jl & 4) ? ~0u : 0u,
                          (jl & 8) ? ~0u : 0u};  // pick() masks

  // Query operand B of the score product: lane l holds head hh, elements
  // kd_index(i, R, 0..7). The descriptor covers only this group's hcnt query
  // rows; head columns past them (and dead columns, sent to row 16) read
  // zeros and are never emitted.
  h8_t qb[F::NKI];
  {
    const rsrc_t rQ = make_rsrc(p.q + qrow0 * D, (uint32_t)hcnt * D * 2);
    const uint32_t qrow = live ? (uint32_t)hh : 16u;
#pragma unroll
    for (int i = 0; i < F::NKI; ++i) qb[i] = F::qfrag(rQ, qrow * D, i, R);
  }
  // bf16 products take the fp16 query as two bf16 operands, q = hi + lo
  // exactly (hi holds 8 of q's 11 significant bits, lo the rest); int8 / int4
  // scores come out of the matrix cores as 2^-24 (q.k + BIAS sum(q)) over the
  // query as the operands carry it, qbias = BIAS sum(q) of the lane's column
  // (zero for fp16). Both need the query's values: formed here, the wait for
  // the query puts a memory round trip ahead of the first K load, so LAZY
  // forms them in the first pass once its K / V loads are out (same-box A/B:
  // int8 / int4 MHA at B 8, N 4096, D 128 6.59 -> 6.10 / 5.81 -> 5.36 us, at
  // B 32, N 512 6.39 -> 6.07 / 6.06 -> 5.67 us; split-K at N 16384 10.97 ->
  // 10.83 / 8.68 -> 8.51 us; B 256 and 2048, several passes a wave: eager).
  bf8_t qhi[F::BF16 ? F::NKI : 1], qlo[F::BF16 ? F::NKI : 1];
  float qbias = 0.0f;
  constexpr bool QPREP = F::BF16 || F::BIASED;
  bool qready = !LAZY;
  auto qprep = [&]() {
    if constexpr (F::BF16) {
#pragma unroll
      for (int i = 0; i < F::NKI; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = (float)qb[i][e];
          qhi[i][e] = (__bf16)f;
          qlo[i][e] = (__bf16)(f - (float)qhi[i][e]);
        }
    }
    if constexpr (F::BIASED) {
      float qs = 0.0f;
#pragma unroll
      for (int i = 0; i < F::NKI; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) qs += (float)qb[i][e] * (16777216.0f / F::kunit(e));
      qbias = F::BIAS * rows4_sum(qs);
    }
  };
  if constexpr (QPREP && !LAZY) qprep();

  float m_run = -INFINITY, l_run = 0.0f;  // of column n, over the tokens this lane scored
  float w_run = 0.0f;  // int8 / int4: sum of the lane's PV weights, in acc's units
  int acc_shift = 0;                      // acc holds the true accumulators times 2^acc_shift
  f4_t acc[VE];                           // O^T: step c, reg k = head-dim VE (4R + k) + c of column n
#pragma unroll
  for (int c = 0; c < VE; ++c) acc[c] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // PVV: head h, element VE n + c, over the lane's tokens 4R .. 4R+3 of every tile
  float accv[PVV ? HG : 1][PVV ? VE : 1];
#pragma unroll
  for (int h = 0; h < (PVV ? HG : 1); ++h)
#pragma unroll
    for (int c = 0; c < (PVV ? VE : 1); ++c) accv[h][c] = 0.0f;
  // PVV: the wave's weights, [tile][token][head] fp32, after its K staging rows
  float* s_pw = nullptr;
  if constexpr (PVV) s_pw = reinterpret_cast<float*>(s_kstage + nw * F::KSTAGE) + w * (U * 16 * HG);

  // Buffer descriptors end at the split's last token, so rows past it read
  // as zeros (their scores are masked); offsets are 32-bit from the row block.
  // Paged rows get a descriptor per tile instead (a tile never crosses a
  // page), ending at the tile's last valid token; a tile whose page id is out
  // of range gets an empty descriptor and its tokens are masked. (Per-tile
  // descriptors for contiguous rows too would spare the vector address adds
  // but put scalar work ahead of every pass's first load: measured slower.)
  const uint32_t sts = 2u * (uint32_t)p.sc_ts;  // scale stride in bytes
  const rsrc_t rK = make_rsrc(Kr, PAGED ? 0u : (uint32_t)hi * ts);
  const rsrc_t rV = make_rsrc(Vr, PAGED ? 0u : (uint32_t)hi * ts);
  const rsrc_t rKs = make_rsrc(Ksr, PAGED ? 0u : (uint32_t)hi * sts);
  const rsrc_t rVs = make_rsrc(Vsr, PAGED ? 0u : (uint32_t)hi * sts);
  // 2-byte rows (fp16, bf16): lane row R loads V tokens 4R .. 4R+3 itself (load
  // j = token 4R + j), each load still whole row segments; narrower rows load
  // token 4j + R (one load covers four consecutive rows) and trade chunks
  // between lane rows afterwards (exchange_4x4). TPERM instead scores the
  // tile's tokens transposed in groups of four (K operand row 4a + b holds
  // token a + 4b): lane row R's score slot k is then token R + 4k, the token
  // whose V that lane row loaded as chunk k, and P.V takes V as loaded. The K
  // loads of a quad of lanes then touch four cache lines instead of two:
  // int8 / fp8 one-pass waves gain (MHA B 8, N 4096, D 128 6.07 -> 5.86 us,
  // B 32, N 512 6.40 -> 6.14 us, split-K N 512 / 4096 6.02 -> 5.83 / 7.49 ->
  // 7.23 us), multi-pass waves and int4 lose 1-2 %.
  constexpr bool VDIRECT = FMT == KV_F16 || FMT == KV_BF16;
  constexpr bool TPERM = (SHORT || LAZY) && (FMT == KV_I8 || FMT == KV_FP8);
  constexpr int TS = TPERM ? 4 : 1;  // token distance between a lane's score slots
  // K loads: operand-A layout straight from memory, or (fp16) whole rows
  // that go through the wave's LDS rows
  uint32_t koff;
  if constexpr (F::STAGE_K)
    koff = F::krow_lane(lane, ts);
  else
    koff = (uint32_t)(TPERM ? (n >> 2) + 4 * (n & 3) : n) * ts + F::klane(R);
  const uint32_t voff = (uint32_t)(VDIRECT ? 4 * R : R) * ts + (uint32_t)n * VG::VBYTES;
  // tile t's sources: descriptors and the byte offset of its first token
  struct TileSrc {
    rsrc_t k, v, ks, vs;
    uint32_t off, soff;
    bool ok;
  };
  auto tile_src = [&](int tb) -> TileSrc {
    TileSrc t;
    if constexpr (PAGED) {
      const int pg = tb >> p.page_log2;
      const int pid = (tb < hi) ? p.page_table[(size_t)b * p.max_pages + pg] : -1;
      t.ok = pid >= 0 && pid < p.num_pages;
      const int in = tb - (pg << p.page_log2);
      const uint32_t nrow = t.ok ? (uint32_t)min(16, hi - tb) : 0u;
      const size_t kvb = (size_t)(t.ok ? pid : 0) * p.kv_bs + (size_t)in * ts;
      const size_t scb = (size_t)(t.ok ? pid : 0) * p.sc_bs + (size_t)in * p.sc_ts;
      t.k = make_rsrc(Kr + kvb, nrow * ts);
      t.v = make_rsrc(Vr + kvb, nrow * ts);
      t.ks = make_rsrc(F::QUANT ? Ksr + scb : nullptr, nrow * sts);
      t.vs = make_rsrc(F::QUANT ? Vsr + scb : nullptr, nrow * sts);
      t.off = 0;
      t.soff = 0;
    } else {
      t.k = rK;
      t.v = rV;
      t.ks = rKs;
      t.vs = rVs;
      t.off = (uint32_t)tb * ts;
      t.soff = (uint32_t)tb * sts;
      t.ok = true;
    }
    return t;
  };

  // Each pass covers U tiles of this wave (tiles interleave across waves).
  // All K loads of the pass are issued, then all V loads, before anything is
  // consumed: straight-line code, so the load counter waits exactly for the
  // data about to be used while the rest is still arriving. The pass scores
  // its U tiles with the matrix cores (S^T: tokens on M, columns on N), keeps
  // in column n the scores of tile jl of each group of P tiles, takes ONE
  // online-softmax step over the pass, and accumulates O^T += V^T P^T on the
  // matrix cores: the packed score layout (lane: column n, score slots k = tokens 4R + k) is
  // operand B of the PV product of tile jl, zero for the group's other tiles,
  // so column n of O^T gathers tile jl's share of head hh.
  const int step = 16 * nw;
  const int slot0 = TPERM ? R : 4 * R;       // token of the lane's score slot 0 in its tile
  const int lane_tok = jl * step + slot0;  // ... from the base of the lane's group of tiles
  // scales of paged rows come through per-tile descriptors: every tile's are
  // loaded and the lane's tile is picked afterwards
  constexpr bool PICK_SC = F::QUANT && PAGED && P > 1;
  // contiguous, 8-byte aligned scale rows: a lane's four scales (tokens 4R ..
  // 4R + 3, a multiple of 4 from lo) are one 8-byte load in passes that lie
  // wholly before hi (past the descriptor's end a load reads zeros dword by
  // dword, so a dword holding a valid and an invalid scale could lose both)
  const bool vec_sc = F::QUANT && !TPERM && !PAGED && sts == 2u && (lo & 3) == 0 &&
                      ((reinterpret_cast<uintptr_t>(Ksr) | reinterpret_cast<uintptr_t>(Vsr)) & 7u) == 0;
  for (int pb = lo + 16 * w; pb < hi; pb += U * step) {
    typename F::KT kr[U][F::KL];
    uint32_t vr[U][4][VD];
    // per-token scales (int8 / int4) of the tokens of the lane's score slots k in its tile of group g
    _Float16 ks[NG][4], vs[NG][4];
    _Float16 kt[PICK_SC ? U : 1][4], vt[PICK_SC ? U : 1][4];
    TileSrc src[U];
#pragma unroll
    for (int u = 0; u < U; ++u) src[u] = tile_src(pb + u * step);
    const bool full = !PAGED && pb + (U - 1) * step + 16 <= hi;  // every token of the pass is before hi
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (F::STAGE_K)
        F::load_k_rows(src[u].k, koff + (F::SOFF_TILE ? 0u : src[u].off), ts, kr[u], F::SOFF_TILE ? src[u].off : 0u);
      else
        F::load_k(src[u].k, koff + (F::SOFF_TILE ? 0u : src[u].off), kr[u], F::SOFF_TILE ? src[u].off : 0u);
    }
    // contiguous rows: with LAZY the scale loads' raw dwords, unpacked once
    // the V loads are out too (unpacked here, a pass waits for its K loads and
    // scales before its V loads leave)
    const bool vec_now = vec_sc && full;  // wave-uniform
    u2_t ksa[F::QUANT && !PAGED && LAZY ? NG : 1], vsa[F::QUANT && !PAGED && LAZY ? NG : 1];
    if constexpr (F::QUANT) {
      if constexpr (!PAGED) {
        if (vec_now) {
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const uint32_t so = (uint32_t)(pb + g * P * step) * 2u;  // wave-uniform
            const uint32_t vo = (uint32_t)lane_tok * 2u + (F::SOFF_TILE ? 0u : so);
            if constexpr (LAZY) {
              ksa[g] = buf_load<8>(rKs, vo, F::SOFF_TILE ? so : 0u);
              vsa[g] = buf_load<8>(rVs, vo, F::SOFF_TILE ? so : 0u);
            } else {
              const u2_t a = buf_load<8>(rKs, vo, F::SOFF_TILE ? so : 0u);
              const u2_t c = buf_load<8>(rVs, vo, F::SOFF_TILE ? so : 0u);
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                ks[g][k] = __builtin_bit_cast(_Float16, (uint16_t)(a[k / 2] >> (16 * (k % 2))));
                vs[g][k] = __builtin_bit_cast(_Float16, (uint16_t)(c[k / 2] >> (16 * (k % 2))));
              }
            }
          }
        } else {
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const uint32_t so = (uint32_t)(pb + g * P * step) * sts;  // wave-uniform
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const uint32_t vo = (uint32_t)(lane_tok + TS * k) * sts + (F::SOFF_TILE ? 0u : so);
              ks[g][k] = __builtin_bit_cast(_Float16, buf_load<2>(rKs, vo, F::SOFF_TILE ? so : 0u));
              vs[g][k] = __builtin_bit_cast(_Float16, buf_load<2>(rVs, vo, F::SOFF_TILE ? so : 0u));
            }
          }
        }
      } else {
        constexpr int T = PICK_SC ? U : NG;  // P == 1 otherwise: tile g is group g
#pragma unroll
        for (int u = 0; u < T; ++u)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t so = src[u].soff + (uint32_t)(slot0 + TS * k) * sts;
            const _Float16 a = __builtin_bit_cast(_Float16, buf_load<2>(src[u].ks, so));
            const _Float16 c = __builtin_bit_cast(_Float16, buf_load<2>(src[u].vs, so));
            if constexpr (PICK_SC) {
              kt[u][k] = a;
              vt[u][k] = c;
            } else {
              ks[u][k] = a;
              vs[u][k] = c;
            }
          }
      }
    } else {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) ks[g][k] = vs[g][k] = (_Float16)1.0f;
    }
    // paged and token-major int4 V without the non-temporal hint: there the 64-byte rows of
    // two KV heads share each cache line, read in turn by workgroups on one XCD (paged, batch 8,
    // N 32768: 68.6 -> 55.1 us; head-major pages flat). Everywhere else the hint is faster
    // (without it int8 / int4 MHA at B 2048 +10 %, paged int8 +18 %).
    constexpr int VCP = (FMT == KV_I4 && (PAGED || KEEPV)) ? 0 : CPOL_NT;
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        load_vchunk<VG::VBYTES, VD, VCP>(src[u].v, voff + (uint32_t)(VDIRECT ? j : 4 * j) * ts + (F::SOFF_TILE ? 0u : src[u].off),
                                         vr[u][j], F::SOFF_TILE ? src[u].off : 0u);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the pass ahead of its use
    FQKV_STAMP(1);  // every load of the pass issued
    if constexpr (QPREP && LAZY) {
      if (!qready) {
        qprep();
        qready = true;
      }
    }
    if constexpr (F::QUANT && !PAGED && LAZY) {
      if (vec_now) {
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t a = ksa[g][k / 2], c = vsa[g][k / 2];
            ks[g][k] = __builtin_bit_cast(_Float16, (uint16_t)(a >> (16 * (k % 2))));
            vs[g][k] = __builtin_bit_cast(_Float16, (uint16_t)(c >> (16 * (k % 2))));
          }
      }
    }

    if constexpr (PICK_SC) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          auto bits = [](_Float16 v) { return (uint32_t)__builtin_bit_cast(uint16_t, v); };
          ks[g][k] = __builtin_bit_cast(_Float16, (uint16_t)pick<P>(jm, [&](int j) { return bits(kt[g * P + j][k]); }));
          vs[g][k] = __builtin_bit_cast(_Float16, (uint16_t)pick<P>(jm, [&](int j) { return bits(vt[g * P + j][k]); }));
        }
    }

    f4_t c4[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (F::STAGE_K) F::stage_k(s_kstage + w * F::KSTAGE, lane, kr[u]);
      c4[u] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < F::NKI; ++i) {
        if constexpr (F::BF16) {
          const bf8_t kf = __builtin_bit_cast(bf8_t, F::kfrag(kr[u], i));
          c4[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qhi[i], c4[u], 0, 0, 0);
          c4[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qlo[i], c4[u], 0, 0, 0);
        } else {
          c4[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(F::kfrag(kr[u], i), qb[i], c4[u], 0, 0, 0);
        }
      }
    }

    // scores of the lane's tiles; tokens past the split (or on a bad page)
    // and dead columns are masked
    float x[NG][4];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float raw = pick<P>(jm, [&](int j) { return c4[g * P + j][k]; });
        x[g][k] = (F::BIASED ? fmaf(raw, 16777216.0f, -qbias) : raw) * (float)ks[g][k];
      }
    if (!full) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          bool ok = pb + g * P * step + lane_tok + TS * k < hi;
          if constexpr (PAGED) ok = ok && pick<P>(jm, [&](int j) { return src[g * P + j].ok ? ~0u : 0u; }) != 0u;
          x[g][k] = ok ? x[g][k] : -INFINITY;
        }
    }
    // the running maximum is the same in every lane of a head, so it joins
    // the lane's own maximum before the reduction
    float mx = m_run;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (P * HG < 16) x[g][k] = live ? x[g][k] : -INFINITY;
        mx = fmaxf(mx, x[g][k]);
      }
    const float mn = head_max<HG, P>(mx);
    const float mu = (mn == -INFINITY) ? 0.0f : mn;
    const float alpha = fast_exp2((m_run - mu) * p.c);  // exactly 1 while the maximum holds
    // The PV operand carries each fp32 weight w = p * (V scale) as an fp16
    // pair hi + lo (hi = w' truncated to fp16, lo = fp16(w' - hi)): two matrix-core steps
    // reproduce the weight to ~2^-22 relative, V being exact in fp16. For
    // int8 / int4, w' = w * 2^shift with a power-of-two shift that puts the
    // pass's largest possible weight at most 2^2 under 2^14, so lo stays clear
    // of the fp16 subnormals (small per-token scales would otherwise push it
    // there, against V values up to 127). The shift only changes when the
    // pass's V scales leave that window; l and acc are kept in units of
    // 2^shift and rescaled exactly when it does. fp16 weights (w = p <= 1, V
    // values of unit size) need no shift.
    int shift = 0;
    if constexpr (F::QUANT) {
      float vmax = 0.0f;
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k) vmax = fmaxf(vmax, (float)vs[g][k]);
      // over the pass (dead columns hold scales of the pass's last tile)
      vmax = head_max<HG, P, true>(vmax);
      // vmax < 2^e with e from the exponent field (vmax is a normal fp32)
      const int e = vmax > 0.0f ? (int)((__builtin_bit_cast(uint32_t, vmax) >> 23) & 0xFFu) - 126 : 0;
      const int ideal = 14 - e;
      shift = (acc_shift <= ideal && acc_shift >= ideal - 2) ? acc_shift : ideal;
    }
    // p 2^shift = 2^((x - mu) c + shift), the argument as one multiply-add
    const float arg0 = (float)shift - mu * p.c;
    h4_t phi[NG], plo[NG];
    float psum = 0.0f, wsum = 0.0f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float wv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float pw = fast_exp2(fmaf(x[g][k], p.c, arg0));
        psum += pw;
        wv[k] = F::QUANT ? pw * (float)vs[g][k] : pw;
        if constexpr (F::BIASED) wsum += wv[k];
      }
      if constexpr (PVV) {
        if (live) {
#pragma unroll
          for (int k = 0; k < 4; ++k) s_pw[((g * P + jl) * 16 + 4 * R + k) * HG + hh] = wv[k];
        }
      }
      if constexpr (F::BF16) {
        // bf16 pairs by truncation: hi = the top 16 bits of w (exact as an
        // fp32 value), lo = the top 16 bits of w - hi; |w - hi - lo| < 2^-16 |w|
        uint32_t bh4[4], bl4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          bh4[k] = __builtin_bit_cast(uint32_t, wv[k]) & 0xFFFF0000u;
          bl4[k] = __builtin_bit_cast(uint32_t, wv[k] - __builtin_bit_cast(float, bh4[k]));
        }
        // the high halves of two dwords -> one dword of two bf16 (element 0 low)
        auto hi2 = [](uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); };
        phi[g] = __builtin_bit_cast(h4_t, u2_t{hi2(bh4[0], bh4[1]), hi2(bh4[2], bh4[3])});
        plo[g] = __builtin_bit_cast(h4_t, u2_t{hi2(bl4[0], bl4[1]), hi2(bl4[2], bl4[3])});
      } else {
        // hi through an explicit conversion (round toward zero): converting
        // with a cast lets the compiler fuse the product into a mixed-precision
        // multiply-add for one use and not another, and the two roundings of w
        // to fp16 can differ, leaving hi + lo an fp16 ulp off w
        const h2_t h01 = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(wv[0], wv[1]));
        const h2_t h23 = __builtin_bit_cast(h2_t, __builtin_amdgcn_cvt_pkrtz(wv[2], wv[3]));
        const h2_t l01 = __builtin_bit_cast(
            h2_t, __builtin_amdgcn_cvt_pkrtz(wv[0] - (float)h01.x, wv[1] - (float)h01.y));
        const h2_t l23 = __builtin_bit_cast(
            h2_t, __builtin_amdgcn_cvt_pkrtz(wv[2] - (float)h23.x, wv[3] - (float)h23.y));
        phi[g] = h4_t{h01.x, h01.y, h23.x, h23.y};
        plo[g] = h4_t{l01.x, l01.y, l23.x, l23.y};
      }
    }
    const float acc_alpha = F::QUANT ? __builtin_amdgcn_ldexpf(alpha, shift - acc_shift) : alpha;
    l_run = l_run * acc_alpha + psum;
    if constexpr (F::BIASED) w_run = w_run * acc_alpha + wsum;
    acc_shift = shift;
    // acc needs rescaling only where the maximum or the shift moved and
    // something has been accumulated (acc is all zero while m = -inf)
    if (__builtin_amdgcn_ballot_w64(acc_alpha != 1.0f && m_run != -INFINITY) != 0) {
      if constexpr (PVV) {
        // a lane accumulates every head, so each takes its own head's factor,
        // from lane h (row 0, column h: head h of the pass's first tile); the
        // factors are the same in every lane row
#pragma unroll
        for (int h = 0; h < HG; ++h) {
          const float ah = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc_alpha), h));
#pragma unroll
          for (int c = 0; c < VE; ++c) accv[h][c] *= ah;
        }
      } else {
#pragma unroll
        for (int c = 0; c < VE; ++c) acc[c] *= acc_alpha;
      }
    }
    m_run = mn;
    if constexpr (PVV) {
      // the lane's V after the row exchange: chunk j = token 4R + j, half c of
      // its dwords = element VE n + c; the weights of that token for every
      // head are one LDS broadcast read per row
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (!VDIRECT) {
#pragma unroll
          for (int dw = 0; dw < VD; ++dw) exchange_4x4(vr[u][0][dw], vr[u][1][dw], vr[u][2][dw], vr[u][3][dw]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float wt[HG];
#pragma unroll
          for (int h = 0; h < HG; ++h) wt[h] = s_pw[(u * 16 + 4 * R + j) * HG + h];
#pragma unroll
          for (int c = 0; c < VE; ++c) {
            const uint32_t d2 = vr[u][j][c / 2];
            const float v = (float)__builtin_bit_cast(_Float16, (uint16_t)((c % 2) ? (d2 >> 16) : (d2 & 0xFFFFu)));
#pragma unroll
            for (int h = 0; h < HG; ++h) accv[h][c] = fmaf(v, wt[h], accv[h][c]);
          }
        }
      }
      continue;
    }
    // Two tiles per product: v_mfma_f32_16x16x32_f16 contracts over 32
    // operand slots, lane row R's slots 8R .. 8R+3 taking the tokens of its
    // score slots (4R .. 4R+3; TPERM R, R+4, R+8, R+12) of tile u and
    // 8R+4 .. 8R+7 the same tokens of tile u + 1 (half the matrix-core time of
    // two 16x16x16 products).
    static_assert(U % 2 == 0, "tiles are paired");
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      // operand B of tile t: the weights of the columns that hold tile t
      // (HG (t % P) .. + HG - 1). fp16 moves them down the row to columns
      // 0 .. HG - 1, so every tile of every pass accumulates into the HG
      // columns of O^T that are emitted and no column sum is left for the
      // end (the other columns gather weights of other tiles, never read).
      // int8 / int4 keep them in place, zero elsewhere: their products carry
      // the bias B sum(w) until the end, and one column holding P tiles'
      // biased sums measured a few 1e-4 off in the split scratch.
      auto wts = [&](int t, h4_t& bh, h4_t& bl) {
#pragma unroll
        for (int dw = 0; dw < VD; ++dw) {
          if constexpr (!VDIRECT && !TPERM) exchange_4x4(vr[t][0][dw], vr[t][1][dw], vr[t][2][dw], vr[t][3][dw]);
#pragma unroll
          for (int j = 0; j < 4; ++j) vr[t][j][dw] = F::vprep(vr[t][j][dw]);
        }
        bh = phi[t / P];
        bl = plo[t / P];
        if constexpr (P > 1 && !F::QUANT) {
          const int sh = HG * (t % P);
          const u2_t h2 = __builtin_bit_cast(u2_t, bh), l2 = __builtin_bit_cast(u2_t, bl);
          bh = __builtin_bit_cast(h4_t, u2_t{row_shl(h2.x, sh), row_shl(h2.y, sh)});
          bl = __builtin_bit_cast(h4_t, u2_t{row_shl(l2.x, sh), row_shl(l2.y, sh)});
        } else if constexpr (P > 1) {
          const bool mine = jl == t % P;
          const u2_t h2 = __builtin_bit_cast(u2_t, bh), l2 = __builtin_bit_cast(u2_t, bl);
          bh = __builtin_bit_cast(h4_t, u2_t{mine ? h2.x : 0u, mine ? h2.y : 0u});
          bl = __builtin_bit_cast(h4_t, u2_t{mine ? l2.x : 0u, mine ? l2.y : 0u});
        }
      };
      h4_t bh0, bl0, bh1, bl1;
      wts(u, bh0, bl0);
      wts(u + 1, bh1, bl1);
      const h8_t bh = __builtin_shufflevector(bh0, bh1, 0, 1, 2, 3, 4, 5, 6, 7);
      const h8_t bl = __builtin_shufflevector(bl0, bl1, 0, 1, 2, 3, 4, 5, 6, 7);
      h8_t vf[VE];
#pragma unroll
      for (int c = 0; c < VE; ++c) {
        vf[c] = __builtin_shufflevector(vfrag<FMT, D>(vr[u], c), vfrag<FMT, D>(vr[u + 1], c), 0, 1, 2, 3, 4, 5, 6, 7);
        if constexpr (F::BF16)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8_t, vf[c]),
                                                           __builtin_bit_cast(bf8_t, bh), acc[c], 0, 0, 0);
        else
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[c], bh, acc[c], 0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < VE; ++c) {
        if constexpr (F::BF16)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8_t, vf[c]),
                                                           __builtin_bit_cast(bf8_t, bl), acc[c], 0, 0, 0);
        else
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[c], bl, acc[c], 0, 0, 0);
      }
    }
  }

  FQKV_STAMP(3);  // last pass's P.V products issued
  // ---- wave totals: l over the four lane rows and the P columns of a head
  // (same running max and shift in all of them); O^T rows are disjoint; its
  // columns 0 .. HG - 1 hold every tile (fp16), or the P columns of a head
  // add up (int8 / int4) ----
  if constexpr (F::QUANT) {
    if constexpr (F::BIASED) {
      // acc[c] * vunit = sum w (v + BIAS): take BIAS sum(w) of the column off
      const float wb = F::BIAS * rows4_sum(w_run);
#pragma unroll
      for (int c = 0; c < VE; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[c][k] = fmaf(acc[c][k], F::vunit(c % VG::EPD), -wb);
    }
    l_run = __builtin_amdgcn_ldexpf(l_run, -acc_shift);
  }
  l_run = cols_sum<HG, P>(rows4_sum(l_run));
  if constexpr (P > 1 && F::QUANT) {
#pragma unroll
    for (int c = 0; c < VE; ++c)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[c][k] = cols_sum<HG, P>(acc[c][k]);
  }
  if constexpr (F::QUANT) {
#pragma unroll
    for (int c = 0; c < VE; ++c)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[c][k] = __builtin_amdgcn_ldexpf(acc[c][k], -acc_shift);
  }
  if constexpr (PVV) {
    // sums over the four lane rows: lane n then holds elements VE n .. VE n + VE-1 of every head
#pragma unroll
    for (int h = 0; h < HG; ++h)
#pragma unroll
      for (int c = 0; c < VE; ++c) accv[h][c] = rows4_sum(accv[h][c]);
    if (R == 0) {
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        if (h < hcnt) {
#pragma unroll
          for (int c = 0; c < VE; c += 4)
            *reinterpret_cast<fl4_t*>(&s_o[w][h][VE * n + c]) =
                fl4_t{accv[h][c], accv[h][c + 1], accv[h][c + 2], accv[h][c + 3]};
        }
      }
    }
  }
  if (n < HG && n < hcnt) {
    if constexpr (!PVV) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float* dst = &s_o[w][n][VE * (4 * R + k)];
#pragma unroll
        for (int c = 0; c < VE; c += 4)
          *reinterpret_cast<fl4_t*>(dst + c) = fl4_t{acc[c][k], acc[c + 1][k], acc[c + 2][k], acc[c + 3][k]};
      }
    }
    if (R == 0) {
      s_m[n][w] = m_run;
      s_l[n][w] = l_run;
    }
  }
  FQKV_STAMP(4);  // wave totals written to LDS
  __syncthreads();
  FQKV_STAMP(5);  // wave-merge barrier passed

  // ---- merge the waves, emit output or split scratch ----
  if (nw == 8)
    merge_waves_emit<D, HG, 8>(p, s_o, s_m, s_l, qrow0, hcnt, s);
  else if (nw == 4)
    merge_waves_emit<D, HG, 4>(p, s_o, s_m, s_l, qrow0, hcnt, s);
  else
    merge_waves_emit<D, HG, 2>(p, s_o, s_m, s_l, qrow0, hcnt, s);

  // ---- in-kernel split merge: the last of the S workgroups of this
  // (KV row, head group) merges the S partials of its heads. The partials
  // above were stored at device scope (sc1, past the non-coherent per-XCD
  // L2s); each thread waits for its stores to complete before the barrier,
  // so by the time thread 0 counts the workgroup in, its partials are
  // visible device-wide. The last arriver reads every partial with
  // device-scope loads. No L2 writeback or invalidate is needed, and nobody
  // waits on the counter, so no workgroup can stall.
  //
  // When the host has found that every workgroup of a group runs on one XCD
  // (p.xcd_local: the XCD of a workgroup is fixed by blockIdx.x mod the XCD
  // count, and split-major order gives a group the same residue for every
  // split), that XCD's L2 is coherent for all of them: the partials, the
  // counter and the merge's loads stay in it (workgroup-scope stores write
  // through the CU's L1 to the L2, the store acknowledgements come from the
  // L2, the counter's atomic executes there, and the merge's sc0 loads skip
  // the merging CU's L1), as on a GPU with one L2.
  FQKV_STAMP(6);  // output or partials issued
  if (!p.direct && p.slot >= 0) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* ctr = arrival_counter(p.slot, wsg);
    if (threadIdx.x == 0)
      s_last = (p.xcd_local ? __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                            : __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == p.S - 1;
    __syncthreads();
    FQKV_STAMP(7);  // arrival known
    if (s_last) {
      if (p.xcd_local)
        merge_splits<D, CPOL_SC0>(p.m_part, p.l_part, p.o_part, p.o, qrow0, hcnt, p.S, s_mw, s_mr);
      else
        merge_splits<D, CPOL_SC1>(p.m_part, p.l_part, p.o_part, p.o, qrow0, hcnt, p.S, s_mw, s_mr);
      FQKV_STAMP(9);  // merge done
      // every workgroup of the group has counted in: reset for the next call
      if (threadIdx.x == 0) {
        if (p.xcd_local)
          __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else
          __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  FQKV_STAMP(10);  // end
}

// Two-kernel form of the split merge (decode_attn_gqa_sk_fast.cu:57-94): one
// workgroup per query head. Used when a call cannot take arrival counters.
template <int D>
__global__ void __launch_bounds__(64 * NW_MAX) combine_kernel(const float* __restrict__ m_part,
                                                              const float* __restrict__ l_part,
                                                              const float* __restrict__ o_part,
                                                              _Float16* __restrict__ o, int S) {
  __shared__ __attribute__((aligned(16))) float s_w[NW_MAX][64];
  __shared__ float s_red[NW_MAX][65];
  merge_splits<D, 0>(m_part, l_part, o_part, o, blockIdx.x, 1, S, s_w, s_red);
}

// Dequantise through the kernels' own conversions (K side: int -> fp16
// operand, V side: int -> fp16 operand; each times its unit less the bias is
// the integer), one thread per (token, lane slot).
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
      for (int e = 0; e < 8; ++e) out[t * D + F::kd_index(i, kb, e)] = ((float)b[e] * F::kunit(e) - F::BIAS) * sc;
    }
  } else {
    using VG = VGeom<F::ROWB, D>;
    const int64_t t = g / 16;
    const int i = (int)(g % 16);
    if (t >= tokens) return;
    uint32_t d[VG::VD];
    load_vchunk<VG::VBYTES, VG::VD>(make_rsrc(Kq + t * F::ROWB, F::ROWB), (uint32_t)i * VG::VBYTES, d);
    const float sc = (float)Ks[t];
#pragma unroll
    for (int k = 0; k < VG::VD; ++k) d[k] = F::vprep(d[k]);
#pragma unroll
    for (int c = 0; c < VG::VE; ++c) {
      const h2_t h = F::vpair(d[c / VG::EPD], d[c / VG::EPD], c % VG::EPD);
      out[t * D + VG::VE * i + c] = ((float)h.x * F::vunit(c % VG::EPD) - F::BIAS) * sc;
    }
  }
}

// ------------------------------------------------------------ launchers ----
// XCD period of a device: the workgroups of a launch are dealt to the XCDs
// round-robin by blockIdx.x. A one-time probe records every workgroup's XCC_ID
// (hardware register 20, bits 3:0) over 4096 workgroups; with n the number of
// distinct ids it accepts n >= 2 only if workgroup i sits on the XCD of
// workgroup i mod n (so the first n are on n distinct XCDs); otherwise (a
// register that reads one value, any other order) the split merge keeps its
// device-scope protocol.
constexpr int XCC_PROBE_BLOCKS = 4096;
constexpr int XCC_ID_HWREG = (3 << 11) | 20;  // s_getreg operand: 4 bits at offset 0 of register 20
static __device__ __align__(256) uint32_t g_xcc_ids[XCC_PROBE_BLOCKS];
static std::atomic<int> g_xcd_period[64];  // 0: not probed, -1: not usable, n: period
static std::mutex g_xcd_probe_mu[64];

__global__ void __launch_bounds__(64) xcc_record_kernel(uint32_t* ids) {
  if (threadIdx.x == 0) ids[blockIdx.x] = (uint32_t)__builtin_amdgcn_s_getreg(XCC_ID_HWREG) & 15u;
}

// The period a run of ids shows: n distinct ids repeating with period n, or
// -1 (one id, or any other order).
static int period_of_ids(const uint32_t* ids, int count) {
  bool seen[16] = {};
  int n = 0;
  for (int i = 0; i < count; ++i)
    if (!seen[ids[i] & 15u]) {
      seen[ids[i] & 15u] = true;
      ++n;
    }
  if (n < 2) return -1;
  for (int i = 1; i < n; ++i)
    for (int j = 0; j < i; ++j)
      if (ids[i] == ids[j]) return -1;
  for (int i = n; i < count; ++i)
    if (ids[i] != ids[i % n]) return -1;
  return n;
}

// Probed on the first eager call per device, one thread at a time (a stream
// that is capturing gets 0, the device-scope protocol, and leaves the probe
// for later). It launches the probe kernel and reads the 16 KiB of ids back
// on the caller's stream, so that first call synchronises the stream once;
// the synchronisation runs in this thread's relaxed capture mode, so a stream
// capture in progress on another thread is not invalidated by it. A HIP error
// stores nothing (a later call probes again); FQKV_XCD_LOCAL_MERGE=0 in the
// environment stores -1. Allocates nothing.
static int xcd_period(hipStream_t st) {
  int dev = 0, cur = 0;
  if ((st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev)) != hipSuccess || hipGetDevice(&cur) != hipSuccess ||
      dev != cur || dev < 0 || dev >= 64)
    return 0;
  int known = g_xcd_period[dev].load(std::memory_order_acquire);
  if (known != 0) return known > 0 ? known : 0;
  if (st == hipStreamPerThread) return 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  if (hipStreamGetCaptureInfo(st, &cs, &id) != hipSuccess || cs != hipStreamCaptureStatusNone) return 0;
  std::lock_guard<std::mutex> lock(g_xcd_probe_mu[dev]);
  known = g_xcd_period[dev].load(std::memory_order_acquire);
  if (known != 0) return known > 0 ? known : 0;
  const char* off = getenv("FQKV_XCD_LOCAL_MERGE");
  if (off && off[0] == '0') {
    g_xcd_period[dev].store(-1, std::memory_order_release);
    return 0;
  }
  uint32_t* ids = nullptr;
  static uint32_t host[64][XCC_PROBE_BLOCKS];  // guarded by the device's probe mutex
  if (hipGetSymbolAddress((void**)&ids, HIP_SYMBOL(g_xcc_ids)) != hipSuccess) return 0;
  void* args[] = {&ids};
  if (hipLaunchKernel((const void*)xcc_record_kernel, dim3(XCC_PROBE_BLOCKS), dim3(64), args, 0, st) != hipSuccess)
    return 0;
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return 0;
  const bool copied = hipMemcpyAsync(host[dev], ids, sizeof(host[dev]), hipMemcpyDeviceToHost, st) == hipSuccess &&
                      hipStreamSynchronize(st) == hipSuccess;
  (void)hipThreadExchangeStreamCaptureMode(&mode);  // restores the caller's mode
  if (!copied) return 0;
  const int res = period_of_ids(host[dev], XCC_PROBE_BLOCKS);
  g_xcd_period[dev].store(res, std::memory_order_release);
  return res > 0 ? res : 0;
}

int xcd_period_of(int device) {
  if (device < 0 || device >= 64) return -1;
  return g_xcd_period[device].load(std::memory_order_acquire);
}

static std::atomic<int> g_pv_valu{0};
void set_pv_valu(int on) { g_pv_valu.store(on ? 1 : 0, std::memory_order_relaxed); }

template <int FMT, int D, int HG>
static hipError_t launch_partial_t(const PartialParams& p, int nblocks, int nw, hipStream_t st) {
  // nw is a maximum: a split shorter than one pass of nw waves would leave
  // waves with nothing to load, so take the fewest waves (at least 2) that
  // still cover the split in one pass -- but, when the splits are merged in
  // the kernel, no fewer than the merge has (head, 64-dim block) units, so
  // that every unit keeps a wave of its own.
  {
    const int u = p.page_table ? tiles_per_pass<FMT, D, HG, true, false>() : tiles_per_pass<FMT, D, HG, false, false>();
    const int tiles = (p.chunk + 15) / 16;
    const int units = p.S > 1 ? HG * (D / 64) : 1;
    while (nw > 2 && nw / 2 >= units && (nw / 2) * u >= tiles) nw /= 2;
  }
  size_t lds = 0;
  if constexpr (Fmt<FMT, D>::STAGE_K) lds = (size_t)nw * Fmt<FMT, D>::KSTAGE;
  if constexpr (FMT == KV_F16 && D == 128 && (HG == 1 || HG == 4)) {
    if (!p.page_table && g_pv_valu.load(std::memory_order_relaxed)) {
      lds += (size_t)nw * tiles_per_pass<FMT, D, HG, false, true>() * 16 * HG * sizeof(float);
      hipLaunchKernelGGL((decode_partial_kernel<FMT, D, HG, false, true>), dim3(nblocks), dim3(64 * nw), lds, st, p);
      return hipGetLastError();
    }
  }
  // the formats with query operands or scales to prepare: LAZY when every wave
  // has one four-tile pass (with two-tile passes it measured slower: int8 /
  // int4 split-K at N 4096 +0.27 us, where N 512 gained 0 / 0.25 us)
  constexpr bool LZ = Fmt<FMT, D>::QUANT || FMT == KV_BF16;
  const int tiles = (p.chunk + 15) / 16;
  if (!p.page_table && !(FMT == KV_I4 && p.hg_k)) {
    // at most two tiles per wave: two-tile passes
    if (tiles <= 2 * nw) {
      hipLaunchKernelGGL((decode_partial_kernel<FMT, D, HG, false, false, false, true>), dim3(nblocks),
                         dim3(64 * nw), lds, st, p);
      return hipGetLastError();
    }
    if (LZ && tiles <= tiles_per_pass<FMT, D, HG, false, false>() * nw) {
      hipLaunchKernelGGL((decode_partial_kernel<FMT, D, HG, false, false, false, false, LZ>), dim3(nblocks),
                         dim3(64 * nw), lds, st, p);
      return hipGetLastError();
    }
  }
  if (p.page_table)
    hipLaunchKernelGGL((decode_partial_kernel<FMT, D, HG, true>), dim3(nblocks), dim3(64 * nw), lds, st, p);
  else if (FMT == KV_I4 && p.hg_k)
    hipLaunchKernelGGL((decode_partial_kernel<FMT, D, HG, false, false, FMT == KV_I4>), dim3(nblocks), dim3(64 * nw),
                       lds, st, p);
  else
    hipLaunchKernelGGL((decode_partial_kernel<FMT, D, HG, false>), dim3(nblocks), dim3(64 * nw), lds, st, p);
  return hipGetLastError();
}

template <int FMT, int D>
static hipError_t launch_partial_d(int hg, const PartialParams& p, int nblocks, int nw, hipStream_t st) {
  switch (hg) {
    case 1: return launch_partial_t<FMT, D, 1>(p, nblocks, nw, st);
    case 2: return launch_partial_t<FMT, D, 2>(p, nblocks, nw, st);
    case 4: return launch_partial_t<FMT, D, 4>(p, nblocks, nw, st);
    case 8: return launch_partial_t<FMT, D, 8>(p, nblocks, nw, st);
    case 16: return launch_partial_t<FMT, D, 16>(p, nblocks, nw, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_partial(int fmt, int D, int hg, const PartialParams& params, int nblocks, int nw,
                          hipStream_t st, int* xcd_local) {
  if ((nw != 2 && nw != 4 && nw != 8) || nblocks < 1 || params.S < 1 || params.ngroups < 1 || params.hkv < 1 ||
      nblocks % params.S != 0)
    return hipErrorInvalidValue;
  PartialParams p = params;
  p.split_major = p.S >= 16;
  p.blk_d = p.split_major ? nblocks / p.S : p.S;
  // the splits of group g are blockIdx.x = s * nwsg + g: one XCD for all of
  // them when nwsg is a multiple of the XCD period
  p.xcd_local = 0;
  if (!p.direct && p.slot >= 0 && p.split_major && p.xcd_ok) {
    const int n = xcd_period(st);
    p.xcd_local = n > 0 && (nblocks / p.S) % n == 0;
  }
  if (xcd_local) *xcd_local = p.xcd_local;
  // head grouping: token-major rows (head stride = row bytes), one
  // query-head group per KV row; the heads sharing a 128-byte line of a token
  // (rows under 128 bytes: int4, and int8 at D 64), as many as divide the
  // head count, and whole blocks of them; the distance d between them makes d
  // workgroups' worth of blockIdx a multiple of the 8 XCDs. (Grouping the
  // heads of a whole 1 KiB span instead measured no faster for int8 and
  // 1.4 % slower for fp16, whose rows share no lines.)
  p.hg_k = p.hg_d = 0;
  {
    constexpr int HEAD_SPAN = 128;
    const int64_t nwsg = (int64_t)nblocks / p.S;
    const int d = p.split_major ? 8 : 8 / std::gcd(p.S, 8);
    const int row_bytes = fmt == KV_I4 ? D / 2 : ((fmt == KV_I8 || fmt == KV_FP8) ? D : 2 * D);
    int k = 0;
    while ((2 << k) * row_bytes <= HEAD_SPAN && p.hkv % (2 << k) == 0 && p.kv_ts >= (2 << k) * row_bytes) ++k;
    int ld = 0;
    while ((1 << ld) < d) ++ld;
    if (k > 0 && p.ngroups == 1 && p.kv_hs == row_bytes && nwsg % ((int64_t)1 << (k + ld)) == 0) {
      p.hg_k = k;
      p.hg_d = ld;
    }
  }
  p.div_blk = make_fastdiv((uint32_t)p.blk_d);
  p.div_groups = make_fastdiv((uint32_t)p.ngroups);
  p.div_hkv = make_fastdiv((uint32_t)p.hkv);
  switch (fmt) {
    case KV_F16: return D == 64 ? launch_partial_d<KV_F16, 64>(hg, p, nblocks, nw, st)
                                : launch_partial_d<KV_F16, 128>(hg, p, nblocks, nw, st);
    case KV_I8: return D == 64 ? launch_partial_d<KV_I8, 64>(hg, p, nblocks, nw, st)
                               : launch_partial_d<KV_I8, 128>(hg, p, nblocks, nw, st);
    case KV_I4: return D == 64 ? launch_partial_d<KV_I4, 64>(hg, p, nblocks, nw, st)
                               : launch_partial_d<KV_I4, 128>(hg, p, nblocks, nw, st);
    case KV_BF16: return D == 64 ? launch_partial_d<KV_BF16, 64>(hg, p, nblocks, nw, st)
                                 : launch_partial_d<KV_BF16, 128>(hg, p, nblocks, nw, st);
    case KV_FP8: return D == 64 ? launch_partial_d<KV_FP8, 64>(hg, p, nblocks, nw, st)
                                : launch_partial_d<KV_FP8, 128>(hg, p, nblocks, nw, st);
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
  // path 0: one thread per (token, K lane group); path 1: per (token, V chunk)
  const int64_t threads = tokens * (path == 0 ? 4 : 16);
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
