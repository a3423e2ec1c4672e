// Internal host <-> kernel interface of libfqkv_decode (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fqkv {

constexpr int NW_MAX = 8;  // waves per workgroup the kernels are sized for

// Division by a run-time constant d (1 <= d < 2^31) for numerators below 2^31:
// n / d = (umulhi(n, magic) + n) >> shift with magic = 2^32 (2^shift - d) / d + 1
// and shift = ceil(log2 d) (the round-up method of Granlund and Montgomery);
// umulhi(n, magic) < n, so the sum stays below 2^32.
struct FastDiv {
  uint32_t magic;
  uint32_t shift;
};
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1;
  return FastDiv{(uint32_t)m, l};
}
__device__ __forceinline__ uint32_t fast_div(uint32_t n, FastDiv f) {
  return (__umulhi(n, f.magic) + n) >> f.shift;
}

// Work item of the partial kernel: split s of group wsg = r * ngroups + g,
// with r the KV row (batch * kv_head), g the query-head group (HG heads of
// the G query heads that share KV row r). With 16 or more splits per group
// the split index varies slowest (blockIdx.x = s * nwsg + wsg, nwsg = rows *
// ngroups): workgroups are dealt to the XCDs in turn, so each XCD then
// streams whole KV rows rather than a slice of every row (0.3-0.4 us off
// the batch-1 split-K headline, 2-4 % at N 32K). With fewer splits the
// group index varies slowest (blockIdx.x = wsg * S + s), which measured
// 9-13 % faster for GQA at 2-8 splits.
struct PartialParams {
  const _Float16* q;     // [R * G, D]
  const uint8_t* K;      // [R, N, row_bytes]
  const uint8_t* V;      // [R, N, row_bytes]
  const _Float16* Ks;    // [R, N] (int8 / int4 only)
  const _Float16* Vs;    // [R, N]
  _Float16* o;           // [R * G, D] when direct
  float* m_part;         // [R * G, S] when !direct
  float* l_part;         // [R * G, S]
  float* o_part;         // [R * G, S, D]
  int G;                 // query heads per KV row
  int N;                 // tokens
  int S;                 // splits
  int chunk;             // ceil(N / S)
  int ngroups;           // ceil(G / HG)
  float c;               // softmax scale * log2(e)
  float scale;           // softmax scale (natural-log units for m_part)
  int direct;            // 1: S == 1, write normalised fp16 output
  int slot;              // !direct: arrival-counter slot for the in-kernel merge, -1 = none
  int xcd_ok;            // set by the caller: the stream may take the XCD-local merge (no CU mask)
  int xcd_local;         // set by launch_partial: every split of a group runs on one XCD
  // KV layout: row r = (b, h) = (r / hkv, r % hkv) starts at K + b*kv_bs + h*kv_hs
  // and its tokens are kv_ts bytes apart; scales likewise in elements. Paged
  // (page_table != null): b indexes page_table [B, max_pages] and seq_lens [B];
  // kv_bs / sc_bs are then the page strides and token t of row r lies in page
  // page_table[b][t >> page_log2] at in-page position t & (2^page_log2 - 1).
  int hkv;
  int64_t kv_bs, kv_hs;
  int kv_ts;
  int64_t sc_bs, sc_hs;
  int sc_ts;
  const int* page_table;
  const int* seq_lens;
  int max_pages;
  int page_log2;
  int num_pages;
  // set by launch_partial from S, ngroups and hkv
  int split_major;  // blockIdx.x = s * nwsg + wsg (else wsg * S + s)
  int blk_d;        // the divisor of that decomposition: nwsg or S
  FastDiv div_blk, div_groups, div_hkv;
  // Head grouping (hg_k = 0: off): in a token-major layout the rows of 2^hg_k
  // neighbouring KV heads share each 128-byte line of a token (two 64-byte
  // int4 rows at D 128). Group wsg is then renumbered so those heads' work
  // items lie 2^hg_d apart in group order, which the round-robin dealing of
  // workgroups to the 8 XCDs puts on one XCD at about the same time: all but
  // the first read the span from that XCD's L2. Only the order of work
  // changes, so results do not depend on where workgroups run.
  int hg_k, hg_d;   // log2 heads per span, log2 distance between them in group order
};

// The reference's contiguous layout: K, V [rows, N, row_bytes], scales [rows, N].
inline void set_contiguous_layout(PartialParams& p, int64_t rows, int64_t N, int row_bytes) {
  p.hkv = (int)rows;
  p.kv_bs = 0;
  p.kv_hs = N * row_bytes;
  p.kv_ts = row_bytes;
  p.sc_bs = 0;
  p.sc_hs = N;
  p.sc_ts = 1;
  p.page_table = nullptr;
  p.seq_lens = nullptr;
  p.max_pages = 0;
  p.page_log2 = 0;
  p.num_pages = 0;
}

// In-kernel split merge: each call with S > 1 takes one of SPLIT_SLOTS slots
// of MAX_SPLIT_GROUPS arrival counters (one per (KV row, head group)).
constexpr int SPLIT_SLOTS = 128;
constexpr int MAX_SPLIT_GROUPS = 16384;

// *xcd_local (optional) receives whether the in-kernel split merge of this
// launch meets in one XCD's L2 (1) or at device scope (0).
hipError_t launch_partial(int fmt, int D, int hg, const PartialParams& p, int nblocks, int nw,
                          hipStream_t st, int* xcd_local = nullptr);
// XCD period of a device as probed (> 0), 0 while not probed (or after a
// probe that a HIP error cut short: it runs again on a later call), -1 when
// the probe found no usable round-robin order.
int xcd_period_of(int device);
hipError_t launch_combine(int D, const float* m_part, const float* l_part, const float* o_part,
                          void* o, int H, int S, int nw, hipStream_t st);
hipError_t launch_dequant(int fmt, int D, int path, const void* Kq, const void* Ks, float* out,
                          int64_t tokens, hipStream_t st);
hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, hipStream_t st);
hipError_t launch_buffer_range(const void* buf, int records, uint32_t* out, hipStream_t st);
// Measurement knob: P.V of fp16, D 128, 1 or 4 heads per group, contiguous rows on the vector ALUs.
void set_pv_valu(int on);
hipError_t launch_quantize(int src, int fmt, int D, const void* X, void* Q, void* S, int64_t tokens,
                           hipStream_t st);
hipError_t launch_quantize_append(int src, int fmt, int D, const void* Xk, const void* Xv, void* Qk, void* Qv,
                                  void* Sk, void* Sv, int64_t rows, int64_t n, int64_t cap, int64_t pos,
                                  const int32_t* pos_of, int64_t rows_per_pos, hipStream_t st);
hipError_t launch_quantize_pages(int src, int fmt, int D, const void* Xk, const void* Xv, const int32_t* slots,
                                 int64_t tokens, int64_t heads, void* Qk, void* Qv, void* Sk, void* Sv,
                                 int64_t num_pages, int page_log2, int64_t q_page, int64_t q_tok, int64_t q_head,
                                 int64_t s_page, int64_t s_tok, int64_t s_head, hipStream_t st);

}  // namespace fqkv
