// extern "C" entry points of libfqkv_decode.so (declared in include/fqkv_decode.h).
//
// Each entry point validates its arguments before touching the GPU, picks
// the query-head group size and split count, and launches the partial
// kernel (plus the combine kernel when the sequence is split) on the
// caller's stream. Nothing here allocates device memory.
#include <hip/hip_runtime.h>
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

#include "fqkv_decode.h"
#include "kv_formats.h"
#include "launch.h"

using namespace fqkv;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FQKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

constexpr int MAX_DEV = 64;

// Split merge: in-kernel (one kernel per call) unless forced to the
// two-kernel form, the call does not fit a slot, or no slot is free.
//
// A slot (a set of arrival counters, one per device) may serve only calls
// that never run at the same time, because the kernel of a call leaves its
// counters at zero only when it ends. Calls on one stream run in order, so
// each stream keeps one slot for its eager calls (EAGER_SLOTS of them, first
// come first served), and each stream of a capture takes a slot of its own
// that eager calls never use (the captured graph replays that slot, so two
// replays of one graph must not overlap -- they would share the caller's
// scratch and output too). Streams or captures beyond the free slots, and the
// per-thread default stream (one handle for many streams), get the
// two-kernel merge, which uses no library state.
std::atomic<int> g_force_two_kernel{0};
// slots 0 .. 11 for eager calls, 12 .. 127 for captures (an engine that captures a graph
// per batch size keeps the one-kernel merge in every graph); 64 KiB of counters each
constexpr int EAGER_SLOTS = 12;

// A slot's stream: its slot, and whether its workgroups may use the XCD-local
// merge (a stream created with a CU mask that leaves CUs out may deal
// workgroups to XCDs in another order, so it keeps the device-scope merge).
struct SlotEntry {
  hipStream_t stream;
  unsigned long long capture;  // capture id (captured slots)
  int slot;
  int xcd_ok;
};
struct SlotTable {
  std::mutex mu;
  std::vector<SlotEntry> eager;
  std::vector<SlotEntry> captured;
};
SlotTable g_slot_tables[MAX_DEV];

// Calls that wanted the in-kernel merge but found every slot of their kind
// taken, and so took the two-kernel merge.
std::atomic<int64_t> g_slot_fallbacks{0};
// The merge protocol of the calling thread's last call (FQKV_MERGE_*).
thread_local int g_last_protocol = FQKV_MERGE_NONE;

// 1 when the stream's CU mask (hipExtStreamGetCUMask) covers as many CUs as
// the device has, 0 when it leaves some out or cannot be read. The null
// stream has no CU mask of its own.
int stream_full_cu_mask(hipStream_t st, int dev) {
  if (st == nullptr) return 1;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
  uint32_t mask[32] = {};
  const uint32_t words = (uint32_t)((cus + 31) / 32);
  if (words > 32 || hipExtStreamGetCUMask(st, words, mask) != hipSuccess) return 0;
  int set = 0;
  for (uint32_t i = 0; i < words; ++i) set += __builtin_popcount(mask[i]);
  return set >= cus;
}

// Slot of a call with `groups` (KV row, head group) pairs on stream st, or -1
// (two-kernel merge); *xcd_ok receives whether the stream may take the
// XCD-local merge. Eager slots are keyed by stream, captured ones by (capture
// id, stream): streams that joined one capture through event waits report the
// same capture id, and their nodes may run side by side on replay, while the
// nodes captured from one stream are ordered.
int merge_slot(hipStream_t st, int64_t groups, int* xcd_ok) {
  *xcd_ok = 0;
  if (g_force_two_kernel.load(std::memory_order_relaxed) || groups > MAX_SPLIT_GROUPS) return -1;
  if (st == hipStreamPerThread) return -1;
  int dev = 0;
  if (st ? hipStreamGetDevice(st, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) return -1;
  if (dev < 0 || dev >= MAX_DEV) return -1;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  if (hipStreamGetCaptureInfo(st, &cs, &id) != hipSuccess) return -1;
  if (cs != hipStreamCaptureStatusNone && cs != hipStreamCaptureStatusActive)
    return -1;  // invalidated capture: the launch fails anyway
  SlotTable& t = g_slot_tables[dev];
  std::lock_guard<std::mutex> lock(t.mu);
  const bool cap = cs == hipStreamCaptureStatusActive;
  std::vector<SlotEntry>& v = cap ? t.captured : t.eager;
  for (const auto& e : v)
    if (e.stream == st && (!cap || e.capture == id)) {
      *xcd_ok = e.xcd_ok;
      return e.slot;
    }
  if ((int)v.size() >= (cap ? SPLIT_SLOTS - EAGER_SLOTS : EAGER_SLOTS)) {
    g_slot_fallbacks.fetch_add(1, std::memory_order_relaxed);
    return -1;
  }
  SlotEntry e{st, cap ? id : 0ull, (cap ? EAGER_SLOTS : 0) + (int)v.size(), stream_full_cu_mask(st, dev)};
  v.push_back(e);
  *xcd_ok = e.xcd_ok;
  return e.slot;
}

int record_protocol(int S, int slot, int xcd_local) {
  g_last_protocol = S <= 1 ? FQKV_MERGE_NONE
                           : (slot < 0 ? FQKV_MERGE_TWO_KERNEL : (xcd_local ? FQKV_MERGE_XCD_LOCAL : FQKV_MERGE_DEVICE));
  return g_last_protocol;
}

// CU count per device, queried once (256 on MI355X).
std::atomic<int> g_cus[MAX_DEV];

int device_cus(int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= MAX_DEV) return fail(FQKV_ERR_HIP, "device index %d out of range", dev);
  int c = g_cus[dev].load(std::memory_order_relaxed);
  if (c <= 0) {
    e = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
    g_cus[dev].store(c, std::memory_order_relaxed);
  }
  *out = c;
  return FQKV_OK;
}

// Query heads per workgroup: the transposed-score kernels carry up to 16
// heads in one matrix-core tile at the same cost, so a group takes all of
// its KV row's query heads up to 16.
int choose_hg(int64_t G, int fmt) {
  (void)fmt;
  if (G <= 1) return 1;
  if (G == 2) return 2;
  if (G <= 4) return 4;
  if (G <= 8) return 8;
  return 16;
}

// Splits for the single-block entry points: about one workgroup per CU, each
// split at least 32 tokens long (measured on MI355X over batch 1..256,
// N 512..16K, G 1 and 4, W 4 and 8: more workgroups than CUs only adds merge
// work; with two-tile passes for short splits, 32-token splits beat 64-token
// ones where the cap binds: GQA B 1, N 512, D 64 5.16 -> 4.51 us).
int64_t splits_for(int64_t rows, int64_t G, int64_t N, int fmt, int64_t W, int cus) {
  (void)W;
  const int hg = choose_hg(G, fmt);
  const int64_t groups = rows * ((G + hg - 1) / hg);
  const int64_t target = (int64_t)cus;
  if (groups >= target) return 1;
  int64_t S = (target + groups - 1) / groups;
  const int64_t cap = N / 32;
  if (S > cap) S = cap;
  return S < 1 ? 1 : S;
}

// Internal split scratch: m [heads*S], l [heads*S], then acc [heads*S*D]
// starting on a 16-byte boundary, so every partial row is 16-byte aligned.
size_t acc_offset_floats(int64_t heads, int64_t S) { return (size_t)((2 * heads * S + 3) & ~(int64_t)3); }
size_t scratch_bytes(int64_t heads, int64_t S, int64_t D) {
  return (acc_offset_floats(heads, S) + (size_t)heads * (size_t)S * (size_t)D) * sizeof(float);
}

int check_common(int64_t N, int64_t D, int64_t W) {
  if (N < 1 || N > INT_MAX - 1024) return fail(FQKV_ERR_ARG, "N: sequence length must be in [1, 2^31 - 1024), got %lld", (long long)N);
  if (D != 64 && D != 128) return fail(FQKV_ERR_ARG, "D: head_dim must be 64 or 128, got %lld", (long long)D);
  if (W != 2 && W != 4 && W != 8) return fail(FQKV_ERR_ARG, "W: waves per workgroup must be 2, 4 or 8, got %lld", (long long)W);
  return FQKV_OK;
}

// Single-block style decode: rows KV rows, G query heads per row. Splits the
// sequence internally when rows alone cannot fill the GPU and the workspace allows.
int64_t row_bytes_of(int fmt, int64_t D) {
  return (fmt == KV_F16 || fmt == KV_BF16) ? 2 * D : (fmt == KV_I4 ? D / 2 : D);
}
// int8 / int4 / fp8: codes with per-token scales
bool is_quant(int fmt) { return fmt == KV_I8 || fmt == KV_I4 || fmt == KV_FP8; }

// KV layout of a single-block call (null: the reference's contiguous layout).
struct Layout {
  int64_t hkv;
  int64_t kv_bs, kv_hs, kv_ts;
  int64_t sc_bs, sc_hs, sc_ts;
  const int* page_table;
  const int* seq_lens;
  int64_t max_pages, page_log2, num_pages;
};

int run_decode(int fmt, const void* q, const void* K, const void* V, const void* Ks,
               const void* Vs, void* o, int64_t rows, int64_t G, int64_t N, int64_t D, int64_t W,
               void* ws, size_t ws_bytes, hipStream_t st, const Layout* L = nullptr) {
  int cus = 0;
  int rc = device_cus(&cus);
  if (rc) return rc;
  const int hg = choose_hg(G, fmt);
  const int64_t ngroups = (G + hg - 1) / hg;
  const int64_t heads = rows * G;
  int64_t S = splits_for(rows, G, N, fmt, W, cus);
  if (S > 1 && (ws == nullptr || scratch_bytes(heads, S, D) > ws_bytes)) {
    int64_t fit = ws ? (int64_t)(ws_bytes / scratch_bytes(heads, 1, D)) : 0;
    while (fit >= 2 && scratch_bytes(heads, fit, D) > ws_bytes) --fit;
    S = fit >= 2 ? (fit < S ? fit : S) : 1;
  }
  if (S > 1 && !aligned(ws, 16)) return fail(FQKV_ERR_ARG, "workspace must be 16-byte aligned");
  const int64_t nblocks = rows * ngroups * S;
  if (nblocks > INT_MAX) return fail(FQKV_ERR_ARG, "problem too large: %lld workgroups", (long long)nblocks);

  PartialParams p{};
  p.q = (const _Float16*)q;
  p.K = (const uint8_t*)K;
  p.V = (const uint8_t*)V;
  p.Ks = (const _Float16*)Ks;
  p.Vs = (const _Float16*)Vs;
  p.o = (_Float16*)o;
  p.G = (int)G;
  p.N = (int)N;
  p.S = (int)S;
  p.chunk = (int)((N + S - 1) / S);
  if (L && L->page_table) p.chunk = (p.chunk + 15) & ~15;  // a paged tile must not cross a page
  p.ngroups = (int)ngroups;
  p.scale = 1.0f / sqrtf((float)D);
  p.c = p.scale * 1.4426950408889634f;
  p.direct = S == 1;
  p.slot = -1;
  set_contiguous_layout(p, rows, N, (int)row_bytes_of(fmt, D));
  if (L) {
    p.hkv = (int)L->hkv;
    p.kv_bs = L->kv_bs;
    p.kv_hs = L->kv_hs;
    p.kv_ts = (int)L->kv_ts;
    p.sc_bs = L->sc_bs;
    p.sc_hs = L->sc_hs;
    p.sc_ts = (int)L->sc_ts;
    p.page_table = L->page_table;
    p.seq_lens = L->seq_lens;
    p.max_pages = (int)L->max_pages;
    p.page_log2 = (int)L->page_log2;
    p.num_pages = (int)L->num_pages;
  }
  if (!p.direct) {
    float* f = (float*)ws;
    p.m_part = f;
    p.l_part = f + heads * S;
    p.o_part = f + acc_offset_floats(heads, S);
    p.slot = merge_slot(st, rows * ngroups, &p.xcd_ok);
  }
  // Workgroups of 4 waves with four times as many work items as CUs, and
  // with more unsplit work items than CUs for rows under 256 bytes (128-byte
  // rows from one per CU on): several share a CU and hide each other's
  // memory latency, where 8-wave ones fit one per CU at these kernels'
  // register counts and leave a partial round (same-box A/B on MI355X at
  // N 4096, 384 / 512 / 768 KV rows: int8 at D 128 -9 / -8 / -6 %, int4
  // -11 / -9 / -9 %, fp8 and int8 at D 64 -8 to -13 %, fp16 at D 64 -13 /
  // -3 / -6 %, int4 at D 64 within 3 %; at 256 rows int8 / fp8 at D 128 and
  // fp16 at D 64 -6 to -8 %, while 64-byte rows are faster with 8 waves;
  // fp16 / bf16 rows of 256 bytes run 1-2 % slower with 4 waves and keep 8
  // below 4 x CUs). W is a maximum.
  const int64_t rowb = row_bytes_of(fmt, D);
  const bool many = nblocks >= 4LL * cus ||
                    (S == 1 && rowb < 256 && (nblocks > cus || (rowb == 128 && nblocks == cus)));
  const int64_t nw = (many && W > 4) ? 4 : W;
  int xcd_local = 0;
  hipError_t e = launch_partial(fmt, (int)D, hg, p, (int)nblocks, (int)nw, st, &xcd_local);
  if (e != hipSuccess) return hip_fail(e, "launch: partial kernel");
  record_protocol((int)S, p.slot, xcd_local);
  if (!p.direct && p.slot < 0) {
    e = launch_combine((int)D, p.m_part, p.l_part, p.o_part, o, (int)heads, (int)S, 4, st);
    if (e != hipSuccess) return hip_fail(e, "launch: combine kernel");
  }
  return FQKV_OK;
}

int check_ptrs_kv(const void* q, const void* K, const void* V, const void* o) {
  if (!q || !K || !V || !o) return fail(FQKV_ERR_ARG, "null tensor pointer");
  if (!aligned(K, 16) || !aligned(V, 16)) return fail(FQKV_ERR_ARG, "K and V must be 16-byte aligned");
  if (!aligned(q, 16) || !aligned(o, 2)) return fail(FQKV_ERR_ARG, "q must be 16-byte and o 2-byte aligned");
  return FQKV_OK;
}

int check_ptrs_quant(int fmt, int64_t D, const void* q, const void* K, const void* V, const void* Ks,
                     const void* Vs, const void* o) {
  if (!q || !K || !V || !Ks || !Vs || !o) return fail(FQKV_ERR_ARG, "null tensor pointer");
  const uintptr_t kal = (fmt == KV_I4 && D == 64) ? 8 : 16;
  if (!aligned(K, kal) || !aligned(V, kal)) return fail(FQKV_ERR_ARG, "K and V must be %d-byte aligned", (int)kal);
  if (!aligned(q, 16) || !aligned(o, 2) || !aligned(Ks, 2) || !aligned(Vs, 2))
    return fail(FQKV_ERR_ARG, "q must be 16-byte aligned, o and scales 2-byte aligned");
  return FQKV_OK;
}

// The kernels address a KV row block with 32-bit byte offsets.
int64_t row_bytes_of(int fmt, int64_t D);

// Byte offsets inside a KV row are 32-bit, formed in the kernel as tile offset
// + lane offset (for int4 summed by the load itself, the tile offset in the
// SGPR offset). A pass of a wave addresses up to 8 tiles spaced 16 tokens x 8
// waves apart even where they lie past the end of the row (those loads return
// zeros), so the row plus 8 x 128 + 16 tokens must fit in 4 GiB: then no offset,
// in the kernel or in the load's own sum, reaches 2^32.
constexpr int64_t ROW_SPAN = int64_t(1) << 32;
constexpr int64_t SPAN_MARGIN_TOKENS = 8 * 16 * 8 + 16;
int check_span(int64_t N, int64_t D, int fmt) {
  const int64_t row_bytes = row_bytes_of(fmt, D);
  if ((N + SPAN_MARGIN_TOKENS) * row_bytes > ROW_SPAN)
    return fail(FQKV_ERR_ARG, "N: %lld tokens of %lld bytes exceed the per-row span (4 GiB less %lld tokens)",
                (long long)N, (long long)row_bytes, (long long)SPAN_MARGIN_TOKENS);
  return FQKV_OK;
}

int sk_fast(int fmt, const void* q, const void* K, const void* V, const void* Ks, const void* Vs,
            float* m_part, float* l_part, float* o_part, void* o, int64_t Hq, int64_t Hkv, int64_t N,
            int64_t D, int64_t S, int64_t W, int64_t CW, void* stream, void* ev_begin, void* ev_end) {
  int rc = check_common(N, D, W);
  if (rc) return rc;
  if (CW != 4 && CW != 8) return fail(FQKV_ERR_ARG, "CW: combine waves must be 4 or 8, got %lld", (long long)CW);
  if (S < 1 || S > (1 << 20)) return fail(FQKV_ERR_ARG, "S: split count must be in [1, 2^20], got %lld", (long long)S);
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0)
    return fail(FQKV_ERR_ARG, "heads: Hq (%lld) must be a positive multiple of Hkv (%lld)", (long long)Hq, (long long)Hkv);
  if (!is_quant(fmt)) {
    rc = check_ptrs_kv(q, K, V, o);
  } else {
    rc = check_ptrs_quant(fmt, D, q, K, V, Ks, Vs, o);
  }
  if (rc) return rc;
  if ((rc = check_span(N, D, fmt))) return rc;
  if (!m_part || !l_part || !o_part) return fail(FQKV_ERR_ARG, "null scratch pointer");
  if (!aligned(o_part, 16)) return fail(FQKV_ERR_ARG, "o_part must be 16-byte aligned");
  const int64_t G = Hq / Hkv;
  const int hg = choose_hg(G, fmt);
  const int64_t ngroups = (G + hg - 1) / hg;
  const int64_t nblocks = Hkv * ngroups * S;
  if (nblocks > INT_MAX || Hq > INT_MAX) return fail(FQKV_ERR_ARG, "problem too large");
  hipStream_t st = (hipStream_t)stream;

  PartialParams p{};
  p.q = (const _Float16*)q;
  p.K = (const uint8_t*)K;
  p.V = (const uint8_t*)V;
  p.Ks = (const _Float16*)Ks;
  p.Vs = (const _Float16*)Vs;
  p.m_part = m_part;
  p.l_part = l_part;
  p.o_part = o_part;
  p.G = (int)G;
  p.N = (int)N;
  p.S = (int)S;
  p.chunk = (int)((N + S - 1) / S);
  p.ngroups = (int)ngroups;
  p.scale = 1.0f / sqrtf((float)D);
  p.c = p.scale * 1.4426950408889634f;
  p.o = (_Float16*)o;
  p.direct = 0;
  set_contiguous_layout(p, Hkv, N, (int)row_bytes_of(fmt, D));
  // S == 1 still writes the scratch (the caller asked for it); with one split
  // the partial kernel also writes the output, and no merge is launched.
  p.slot = S > 1 ? merge_slot(st, Hkv * ngroups, &p.xcd_ok) : -1;
  hipError_t e;
  if (ev_begin && (e = hipEventRecord((hipEvent_t)ev_begin, st)) != hipSuccess) return hip_fail(e, "hipEventRecord");
  int xcd_local = 0;
  e = launch_partial(fmt, (int)D, hg, p, (int)nblocks, (int)W, st, &xcd_local);
  if (e != hipSuccess) return hip_fail(e, "partial");
  record_protocol((int)S, p.slot, xcd_local);
  if (ev_end && (e = hipEventRecord((hipEvent_t)ev_end, st)) != hipSuccess) return hip_fail(e, "hipEventRecord");
  if (S > 1 && p.slot < 0) {
    e = launch_combine((int)D, m_part, l_part, o_part, o, (int)Hq, (int)S, (int)CW, st);
    if (e != hipSuccess) return hip_fail(e, "combine");
  }
  return FQKV_OK;
}

// ---- the no-allocation split-K entry point's scratch ----
//
// fqkv_gqa_sk_fast_noalloc keeps the split partials (m, l, acc) that
// fqkv_gqa_sk_fast takes from the caller in this file-scope device array
// instead: NOALLOC_SCRATCH_BYTES per device, allocated when the code object
// loads and held until the process ends. In host code `scratch` names a
// host-side stand-in, not device memory, so its device address is looked up
// once per device with hipGetSymbolAddress (with that device current) and
// only that address is handed to kernels. Every call on a device shares the
// device's array and leaves its last partials there; nothing in it has to
// start at zero (the partial kernel writes every entry the merge reads).
// Calls that overlap on one device race on it.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEV];

int scratch_address(hipStream_t st, void** out) {
  int dev = 0;
  hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "scratch: device of the stream");
  if (dev < 0 || dev >= MAX_DEV) return fail(FQKV_ERR_HIP, "scratch: device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess && e2 != hipSuccess) e = e2;
    }
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(FQKV_ERR_HIP, "hipGetSymbolAddress(scratch) returned no address");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FQKV_OK;
}

}  // namespace

extern "C" {

const char* fqkv_last_error(void) { return g_err; }

const char* fqkv_version(void) { return "fqkv_decode 0.1.0 (gfx950)"; }

int fqkv_set_pv_valu(int enable) {
  set_pv_valu(enable);
  return FQKV_OK;
}

int fqkv_set_two_kernel_merge(int enable) {
  g_force_two_kernel.store(enable ? 1 : 0, std::memory_order_relaxed);
  return FQKV_OK;
}

int fqkv_last_merge_protocol(void) { return g_last_protocol; }

int64_t fqkv_merge_fallback_count(void) { return g_slot_fallbacks.load(std::memory_order_relaxed); }

int fqkv_xcd_period(int device) { return xcd_period_of(device); }

int fqkv_release_capture_slots(void) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= MAX_DEV) return fail(FQKV_ERR_HIP, "device index %d out of range", dev);
  SlotTable& t = g_slot_tables[dev];
  std::lock_guard<std::mutex> lock(t.mu);
  t.captured.clear();
  return FQKV_OK;
}

int fqkv_device_cu_count(int* cu_count) {
  if (!cu_count) return fail(FQKV_ERR_ARG, "null cu_count");
  return device_cus(cu_count);
}

int64_t fqkv_choose_splits(int64_t rows, int64_t G, int64_t N, int64_t D, int kv_format, int64_t W) {
  (void)D;
  int cus = 256;
  if (device_cus(&cus) != FQKV_OK) cus = 256;
  if (rows < 1 || G < 1 || N < 1) return 1;
  return splits_for(rows, G, N, kv_format, W, cus);
}

size_t fqkv_workspace_bytes(int64_t rows, int64_t G, int64_t N, int64_t D, int kv_format, int64_t W) {
  const int64_t S = fqkv_choose_splits(rows, G, N, D, kv_format, W);
  return S > 1 ? scratch_bytes(rows * G, S, D) : 0;
}

int fqkv_decode_attn_fp16_mw(const void* q, const void* K, const void* V, void* o, int64_t B,
                             int64_t N, int64_t D, int64_t W, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc = check_common(N, D, W);
  if (rc) return rc;
  if (B < 1) return fail(FQKV_ERR_ARG, "B: batch must be >= 1, got %lld", (long long)B);
  if ((rc = check_ptrs_kv(q, K, V, o))) return rc;
  if ((rc = check_span(N, D, KV_F16))) return rc;
  return run_decode(KV_F16, q, K, V, nullptr, nullptr, o, B, 1, N, D, W, workspace, workspace_bytes,
                    (hipStream_t)stream);
}

static int quant_entry(int fmt, const void* q, const void* K, const void* V, const void* Ks,
                       const void* Vs, void* o, int64_t B, int64_t N, int64_t D, int64_t W,
                       void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common(N, D, W);
  if (rc) return rc;
  if (B < 1) return fail(FQKV_ERR_ARG, "B: batch must be >= 1, got %lld", (long long)B);
  if ((rc = check_ptrs_quant(fmt, D, q, K, V, Ks, Vs, o))) return rc;
  if ((rc = check_span(N, D, fmt))) return rc;
  return run_decode(fmt, q, K, V, Ks, Vs, o, B, 1, N, D, W, workspace, workspace_bytes,
                    (hipStream_t)stream);
}

int fqkv_decode_attn_int8_mw(const void* q, const void* K, const void* V, const void* Ks,
                             const void* Vs, void* o, int64_t B, int64_t N, int64_t D,
                             int64_t W, void* workspace, size_t workspace_bytes, void* stream) {
  return quant_entry(KV_I8, q, K, V, Ks, Vs, o, B, N, D, W, workspace, workspace_bytes, stream);
}

int fqkv_decode_attn_int4(const void* q, const void* K, const void* V, const void* Ks,
                          const void* Vs, void* o, int64_t B, int64_t N, int64_t D, int64_t W,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return quant_entry(KV_I4, q, K, V, Ks, Vs, o, B, N, D, W, workspace, workspace_bytes, stream);
}

int fqkv_decode_attn_gqa(const void* q, const void* K, const void* V, void* o, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int64_t W,
                         void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common(N, D, W);
  if (rc) return rc;
  if (B < 1) return fail(FQKV_ERR_ARG, "B: batch must be >= 1, got %lld", (long long)B);
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0)
    return fail(FQKV_ERR_ARG, "heads: Hq (%lld) must be a positive multiple of Hkv (%lld)", (long long)Hq, (long long)Hkv);
  if ((rc = check_ptrs_kv(q, K, V, o))) return rc;
  if ((rc = check_span(N, D, KV_F16))) return rc;
  return run_decode(KV_F16, q, K, V, nullptr, nullptr, o, B * Hkv, Hq / Hkv, N, D, W, workspace,
                    workspace_bytes, (hipStream_t)stream);
}

int fqkv_gqa_sk_fast(const void* q, const void* K, const void* V, float* m_part, float* l_part,
                     float* o_part, void* o, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                     int64_t S, int64_t W, int64_t CW, void* stream) {
  return sk_fast(KV_F16, q, K, V, nullptr, nullptr, m_part, l_part, o_part, o, Hq, Hkv, N, D, S, W, CW,
                 stream, nullptr, nullptr);
}

int fqkv_gqa_sk_fast_timed(const void* q, const void* K, const void* V, float* m_part,
                           float* l_part, float* o_part, void* o, int64_t Hq, int64_t Hkv,
                           int64_t N, int64_t D, int64_t S, int64_t W, int64_t CW, void* stream,
                           void* ev_begin, void* ev_end) {
  return sk_fast(KV_F16, q, K, V, nullptr, nullptr, m_part, l_part, o_part, o, Hq, Hkv, N, D, S, W, CW,
                 stream, ev_begin, ev_end);
}

int fqkv_gqa_sk_fast_noalloc(const void* q, const void* K, const void* V, void* o, int64_t Hq, int64_t Hkv,
                             int64_t N, int64_t D, int64_t S, int64_t W, int64_t CW, void* stream) {
  // the argument checks sk_fast makes before any HIP call, plus the scratch size
  int rc = check_common(N, D, W);
  if (rc) return rc;
  if (S < 1 || S > (1 << 20)) return fail(FQKV_ERR_ARG, "S: split count must be in [1, 2^20], got %lld", (long long)S);
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0)
    return fail(FQKV_ERR_ARG, "heads: Hq (%lld) must be a positive multiple of Hkv (%lld)", (long long)Hq, (long long)Hkv);
  if (Hq > (int64_t(1) << 24))  // keeps the size arithmetic below far from overflow
    return fail(FQKV_ERR_ARG, "heads: Hq (%lld) too large for the no-allocation scratch", (long long)Hq);
  // m [Hq*S], l [Hq*S], then acc [Hq*S*D] from a 16-byte boundary
  const size_t acc_off = (size_t)((2 * Hq * S + 3) & ~(int64_t)3) * sizeof(float);
  const size_t need = acc_off + (size_t)Hq * (size_t)S * (size_t)D * sizeof(float);
  if (need > NOALLOC_SCRATCH_BYTES)
    return fail(FQKV_ERR_ARG, "S: %lld splits of %lld heads need %zu bytes of partials, more than the %zu-byte "
                "no-allocation scratch; use fewer splits or fqkv_gqa_sk_fast", (long long)S, (long long)Hq, need,
                NOALLOC_SCRATCH_BYTES);
  if ((rc = check_ptrs_kv(q, K, V, o))) return rc;
  void* base = nullptr;
  if ((rc = scratch_address((hipStream_t)stream, &base))) return rc;
  float* f = (float*)base;
  return sk_fast(KV_F16, q, K, V, nullptr, nullptr, f, f + Hq * S, (float*)((char*)base + acc_off), o, Hq, Hkv, N, D,
                 S, W, CW, stream, nullptr, nullptr);
}

int fqkv_decode_attn_gqa_quant(const void* q, const void* K, const void* V, const void* Ks,
                               const void* Vs, void* o, int64_t B, int64_t Hq, int64_t Hkv, int64_t N,
                               int64_t D, int kv_format, int64_t W, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (kv_format != FQKV_KV_I8 && kv_format != FQKV_KV_I4 && kv_format != FQKV_KV_FP8)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_I8, FQKV_KV_I4 or FQKV_KV_FP8");
  int rc = check_common(N, D, W);
  if (rc) return rc;
  if (B < 1) return fail(FQKV_ERR_ARG, "B: batch must be >= 1, got %lld", (long long)B);
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0)
    return fail(FQKV_ERR_ARG, "heads: Hq (%lld) must be a positive multiple of Hkv (%lld)", (long long)Hq, (long long)Hkv);
  if ((rc = check_ptrs_quant(kv_format, D, q, K, V, Ks, Vs, o))) return rc;
  if ((rc = check_span(N, D, kv_format))) return rc;
  return run_decode(kv_format, q, K, V, Ks, Vs, o, B * Hkv, Hq / Hkv, N, D, W, workspace,
                    workspace_bytes, (hipStream_t)stream);
}

int fqkv_gqa_sk_fast_quant(const void* q, const void* K, const void* V, const void* Ks, const void* Vs,
                           float* m_part, float* l_part, float* o_part, void* o, int64_t Hq,
                           int64_t Hkv, int64_t N, int64_t D, int kv_format, int64_t S, int64_t W,
                           int64_t CW, void* stream) {
  if (kv_format != FQKV_KV_I8 && kv_format != FQKV_KV_I4 && kv_format != FQKV_KV_FP8 && kv_format != FQKV_KV_BF16)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_I8, FQKV_KV_I4, FQKV_KV_FP8 or FQKV_KV_BF16");
  return sk_fast(kv_format, q, K, V, Ks, Vs, m_part, l_part, o_part, o, Hq, Hkv, N, D, S, W, CW, stream,
                 nullptr, nullptr);
}

static int check_layout_common(int fmt, int64_t D, const void* q, const void* K, const void* V,
                               const void* Ks, const void* Vs, const void* o, int64_t kv_bs, int64_t kv_hs,
                               int64_t kv_ts, int64_t sc_bs, int64_t sc_hs, int64_t sc_ts) {
  if (fmt != FQKV_KV_F16 && fmt != FQKV_KV_I8 && fmt != FQKV_KV_I4 && fmt != FQKV_KV_BF16 && fmt != FQKV_KV_FP8)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_F16, FQKV_KV_BF16, FQKV_KV_I8, FQKV_KV_I4 or FQKV_KV_FP8");
  int rc = !is_quant(fmt) ? check_ptrs_kv(q, K, V, o) : check_ptrs_quant(fmt, D, q, K, V, Ks, Vs, o);
  if (rc) return rc;
  const int64_t rb = row_bytes_of(fmt, D);
  const int64_t al = (fmt == KV_I4 && D == 64) ? 8 : 16;
  if (kv_ts < rb || kv_ts > INT_MAX || kv_ts % al || kv_hs < 0 || kv_hs % al || kv_bs < 0 || kv_bs % al)
    return fail(FQKV_ERR_ARG, "strides: KV token stride must be >= %lld bytes and all KV strides multiples of %lld "
                "bytes, got batch %lld, head %lld, token %lld", (long long)rb, (long long)al, (long long)kv_bs,
                (long long)kv_hs, (long long)kv_ts);
  if (is_quant(fmt) && (sc_ts < 1 || sc_ts > INT_MAX / 2 || sc_hs < 0 || sc_bs < 0))
    return fail(FQKV_ERR_ARG, "strides: scale strides must be non-negative with a token stride >= 1");
  return FQKV_OK;
}

int fqkv_decode_attn_gqa_strided(const void* q, const void* K, const void* V, const void* Ks, const void* Vs,
                                 void* o, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int kv_format,
                                 int64_t kv_batch_stride, int64_t kv_head_stride, int64_t kv_token_stride,
                                 int64_t sc_batch_stride, int64_t sc_head_stride, int64_t sc_token_stride,
                                 int64_t W, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common(N, D, W);
  if (rc) return rc;
  if (B < 1) return fail(FQKV_ERR_ARG, "B: batch must be >= 1, got %lld", (long long)B);
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0)
    return fail(FQKV_ERR_ARG, "heads: Hq (%lld) must be a positive multiple of Hkv (%lld)", (long long)Hq, (long long)Hkv);
  if ((rc = check_layout_common(kv_format, D, q, K, V, Ks, Vs, o, kv_batch_stride, kv_head_stride,
                                kv_token_stride, sc_batch_stride, sc_head_stride, sc_token_stride)))
    return rc;
  if ((N + SPAN_MARGIN_TOKENS) * kv_token_stride > ROW_SPAN ||
      (is_quant(kv_format) && 2 * (N + SPAN_MARGIN_TOKENS) * sc_token_stride > ROW_SPAN))
    return fail(FQKV_ERR_ARG, "N: %lld tokens at a %lld-byte stride exceed the per-row span (4 GiB less %lld tokens)",
                (long long)N, (long long)kv_token_stride, (long long)SPAN_MARGIN_TOKENS);
  Layout L{Hkv, kv_batch_stride, kv_head_stride, kv_token_stride, sc_batch_stride, sc_head_stride, sc_token_stride,
           nullptr, nullptr, 0, 0, 0};
  return run_decode(kv_format, q, K, V, Ks, Vs, o, B * Hkv, Hq / Hkv, N, D, W, workspace, workspace_bytes,
                    (hipStream_t)stream, &L);
}

int fqkv_decode_attn_gqa_paged(const void* q, const void* K_pages, const void* V_pages, const void* Ks_pages,
                               const void* Vs_pages, const int32_t* page_table, const int32_t* seq_lens, void* o,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t num_pages, int64_t max_pages,
                               int64_t page_size, int64_t max_seq_len, int64_t D, int kv_format,
                               int64_t kv_page_stride, int64_t kv_head_stride, int64_t kv_token_stride,
                               int64_t sc_page_stride, int64_t sc_head_stride, int64_t sc_token_stride,
                               int64_t W, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_common(max_seq_len, D, W);
  if (rc) return rc;
  if (B < 1) return fail(FQKV_ERR_ARG, "B: batch must be >= 1, got %lld", (long long)B);
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0)
    return fail(FQKV_ERR_ARG, "heads: Hq (%lld) must be a positive multiple of Hkv (%lld)", (long long)Hq, (long long)Hkv);
  if (page_size < 16 || page_size > (1 << 20) || (page_size & (page_size - 1)))
    return fail(FQKV_ERR_ARG, "page_size: must be a power of two in [16, 2^20], got %lld", (long long)page_size);
  if (num_pages < 1 || num_pages > INT_MAX || max_pages < 1 || max_pages > INT_MAX ||
      max_pages * page_size > INT_MAX - 1024)
    return fail(FQKV_ERR_ARG, "pages: need 1 <= num_pages, max_pages and max_pages * page_size < 2^31 - 1024");
  if (!page_table || !seq_lens) return fail(FQKV_ERR_ARG, "null page table or sequence lengths");
  if (!aligned(page_table, 4) || !aligned(seq_lens, 4)) return fail(FQKV_ERR_ARG, "page table and lengths must be 4-byte aligned");
  if ((rc = check_layout_common(kv_format, D, q, K_pages, V_pages, Ks_pages, Vs_pages, o, kv_page_stride,
                                kv_head_stride, kv_token_stride, sc_page_stride, sc_head_stride, sc_token_stride)))
    return rc;
  if (16 * kv_token_stride > (int64_t)UINT32_MAX)
    return fail(FQKV_ERR_ARG, "strides: token stride too large");
  int64_t lg = 0;
  while ((int64_t(1) << lg) < page_size) ++lg;
  const int64_t N = max_seq_len < max_pages * page_size ? max_seq_len : max_pages * page_size;
  Layout L{Hkv, kv_page_stride, kv_head_stride, kv_token_stride, sc_page_stride, sc_head_stride, sc_token_stride,
           page_table, seq_lens, max_pages, lg, num_pages};
  return run_decode(kv_format, q, K_pages, V_pages, Ks_pages, Vs_pages, o, B * Hkv, Hq / Hkv, N, D, W, workspace,
                    workspace_bytes, (hipStream_t)stream, &L);
}

int fqkv_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, void* stream) {
  if (!src) return fail(FQKV_ERR_ARG, "null source pointer");
  if (bytes == 0 || bytes % 16) return fail(FQKV_ERR_ARG, "bytes: must be a positive multiple of 16, got %zu", bytes);
  if (!aligned(src, 16)) return fail(FQKV_ERR_ARG, "source must be 16-byte aligned");
  if (blocks < 1 || blocks > (1 << 20)) return fail(FQKV_ERR_ARG, "blocks: must be in [1, 2^20], got %d", blocks);
  hipError_t e = launch_stream_read(src, bytes, sink, blocks, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "launch: stream read kernel");
  return FQKV_OK;
}

int fqkv_probe_buffer_range(const void* buf, size_t bytes, int records, uint32_t* out, void* stream) {
  if (!buf || !out) return fail(FQKV_ERR_ARG, "null pointer");
  if (!aligned(buf, 16) || !aligned(out, 4)) return fail(FQKV_ERR_ARG, "buffer must be 16-byte aligned");
  if (records < 16 || records % 16) return fail(FQKV_ERR_ARG, "records: must be a positive multiple of 16, got %d", records);
  if (bytes < (size_t)records + 64)
    return fail(FQKV_ERR_ARG, "bytes: the buffer must extend 64 bytes past records (%d), got %zu", records, bytes);
  hipError_t e = launch_buffer_range(buf, records, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "launch: buffer range probe");
  return FQKV_OK;
}

int fqkv_dequant_kv(const void* Kq, const void* Ks, float* out, int64_t tokens, int64_t D,
                    int kv_format, int path, void* stream) {
  if (kv_format != FQKV_KV_I8 && kv_format != FQKV_KV_I4)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_I8 or FQKV_KV_I4");
  if (D != 64 && D != 128) return fail(FQKV_ERR_ARG, "D: head_dim must be 64 or 128, got %lld", (long long)D);
  if (path != 0 && path != 1) return fail(FQKV_ERR_ARG, "path must be 0 (K side) or 1 (V side)");
  if (tokens < 1) return fail(FQKV_ERR_ARG, "tokens must be >= 1");
  if (!Kq || !Ks || !out) return fail(FQKV_ERR_ARG, "null tensor pointer");
  const uintptr_t kal = (kv_format == FQKV_KV_I4 && D == 64) ? 8 : 16;
  if (!aligned(Kq, kal)) return fail(FQKV_ERR_ARG, "Kq must be %d-byte aligned", (int)kal);
  if (!aligned(Ks, 2) || !aligned(out, 4)) return fail(FQKV_ERR_ARG, "misaligned scale or output pointer");
  hipError_t e = launch_dequant(kv_format, (int)D, path, Kq, Ks, out, tokens, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "launch: dequant kernel");
  return FQKV_OK;
}

int fqkv_quantize_kv(const void* X, int x_dtype, void* Q, void* scales, int64_t tokens, int64_t D,
                     int kv_format, void* stream) {
  if (kv_format != FQKV_KV_I8 && kv_format != FQKV_KV_I4 && kv_format != FQKV_KV_FP8)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_I8, FQKV_KV_I4 or FQKV_KV_FP8");
  if (x_dtype != FQKV_SRC_F16 && x_dtype != FQKV_SRC_F32 && x_dtype != FQKV_SRC_BF16)
    return fail(FQKV_ERR_ARG, "x_dtype must be FQKV_SRC_F16, FQKV_SRC_F32 or FQKV_SRC_BF16");
  if (D != 64 && D != 128) return fail(FQKV_ERR_ARG, "D: head_dim must be 64 or 128, got %lld", (long long)D);
  if (tokens < 1) return fail(FQKV_ERR_ARG, "tokens must be >= 1, got %lld", (long long)tokens);
  if (!X || !Q || !scales) return fail(FQKV_ERR_ARG, "null tensor pointer");
  const uintptr_t xal = (x_dtype != FQKV_SRC_F32 && D == 64) ? 8 : 16;
  const uintptr_t qal = kv_format == FQKV_KV_I4 ? (D == 128 ? 4 : 2) : (D == 128 ? 8 : 4);
  if (!aligned(X, xal)) return fail(FQKV_ERR_ARG, "X must be %d-byte aligned", (int)xal);
  if (!aligned(Q, qal)) return fail(FQKV_ERR_ARG, "Q must be %d-byte aligned", (int)qal);
  if (!aligned(scales, 2)) return fail(FQKV_ERR_ARG, "scales must be 2-byte aligned");
  hipError_t e = launch_quantize(x_dtype, kv_format, (int)D, X, Q, scales, tokens,
                                 (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "launch: quantize kernel");
  return FQKV_OK;
}

int fqkv_quantize_kv_append(const void* K_new, const void* V_new, int x_dtype, void* K_cache, void* V_cache,
                            void* Ks_cache, void* Vs_cache, int64_t rows, int64_t n_new, int64_t capacity,
                            int64_t pos, int64_t D, int kv_format, void* stream) {
  if (kv_format != FQKV_KV_I8 && kv_format != FQKV_KV_I4 && kv_format != FQKV_KV_FP8)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_I8, FQKV_KV_I4 or FQKV_KV_FP8");
  if (x_dtype != FQKV_SRC_F16 && x_dtype != FQKV_SRC_F32 && x_dtype != FQKV_SRC_BF16)
    return fail(FQKV_ERR_ARG, "x_dtype must be FQKV_SRC_F16, FQKV_SRC_F32 or FQKV_SRC_BF16");
  if (D != 64 && D != 128) return fail(FQKV_ERR_ARG, "D: head_dim must be 64 or 128, got %lld", (long long)D);
  if (rows < 1 || n_new < 1) return fail(FQKV_ERR_ARG, "rows and n_new must be >= 1, got %lld and %lld",
                                         (long long)rows, (long long)n_new);
  if (pos < 0 || capacity < 1 || n_new > capacity - pos)
    return fail(FQKV_ERR_ARG, "pos: tokens %lld .. %lld do not fit a capacity of %lld", (long long)pos,
                (long long)(pos + n_new - 1), (long long)capacity);
  if (!K_new || !V_new || !K_cache || !V_cache || !Ks_cache || !Vs_cache) return fail(FQKV_ERR_ARG, "null tensor pointer");
  const uintptr_t xal = (x_dtype != FQKV_SRC_F32 && D == 64) ? 8 : 16;
  const uintptr_t qal = kv_format == FQKV_KV_I4 ? (D == 128 ? 4 : 2) : (D == 128 ? 8 : 4);
  if (!aligned(K_new, xal) || !aligned(V_new, xal)) return fail(FQKV_ERR_ARG, "K_new and V_new must be %d-byte aligned", (int)xal);
  if (!aligned(K_cache, qal) || !aligned(V_cache, qal)) return fail(FQKV_ERR_ARG, "caches must be %d-byte aligned", (int)qal);
  if (!aligned(Ks_cache, 2) || !aligned(Vs_cache, 2)) return fail(FQKV_ERR_ARG, "scales must be 2-byte aligned");
  hipError_t e = launch_quantize_append(x_dtype, kv_format, (int)D, K_new, V_new, K_cache, V_cache,
                                        Ks_cache, Vs_cache, rows, n_new, capacity, pos, nullptr, 1,
                                        (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "launch: quantize append kernel");
  return FQKV_OK;
}

int fqkv_quantize_kv_append_at(const void* K_new, const void* V_new, int x_dtype, void* K_cache, void* V_cache,
                               void* Ks_cache, void* Vs_cache, int64_t rows, int64_t n_new, int64_t capacity,
                               const int32_t* pos, int64_t rows_per_pos, int64_t D, int kv_format, void* stream) {
  if (kv_format != FQKV_KV_I8 && kv_format != FQKV_KV_I4 && kv_format != FQKV_KV_FP8)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_I8, FQKV_KV_I4 or FQKV_KV_FP8");
  if (x_dtype != FQKV_SRC_F16 && x_dtype != FQKV_SRC_F32 && x_dtype != FQKV_SRC_BF16)
    return fail(FQKV_ERR_ARG, "x_dtype must be FQKV_SRC_F16, FQKV_SRC_F32 or FQKV_SRC_BF16");
  if (D != 64 && D != 128) return fail(FQKV_ERR_ARG, "D: head_dim must be 64 or 128, got %lld", (long long)D);
  if (rows < 1 || n_new < 1) return fail(FQKV_ERR_ARG, "rows and n_new must be >= 1, got %lld and %lld",
                                         (long long)rows, (long long)n_new);
  if (capacity < 1 || n_new > capacity)
    return fail(FQKV_ERR_ARG, "pos: %lld new tokens do not fit a capacity of %lld", (long long)n_new,
                (long long)capacity);
  if (rows_per_pos < 1 || rows % rows_per_pos != 0)
    return fail(FQKV_ERR_ARG, "pos: rows_per_pos (%lld) must divide rows (%lld)", (long long)rows_per_pos,
                (long long)rows);
  if (!K_new || !V_new || !K_cache || !V_cache || !Ks_cache || !Vs_cache || !pos)
    return fail(FQKV_ERR_ARG, "null tensor pointer");
  const uintptr_t xal = (x_dtype != FQKV_SRC_F32 && D == 64) ? 8 : 16;
  const uintptr_t qal = kv_format == FQKV_KV_I4 ? (D == 128 ? 4 : 2) : (D == 128 ? 8 : 4);
  if (!aligned(K_new, xal) || !aligned(V_new, xal)) return fail(FQKV_ERR_ARG, "K_new and V_new must be %d-byte aligned", (int)xal);
  if (!aligned(K_cache, qal) || !aligned(V_cache, qal)) return fail(FQKV_ERR_ARG, "caches must be %d-byte aligned", (int)qal);
  if (!aligned(Ks_cache, 2) || !aligned(Vs_cache, 2)) return fail(FQKV_ERR_ARG, "scales must be 2-byte aligned");
  if (!aligned(pos, 4)) return fail(FQKV_ERR_ARG, "pos must be 4-byte aligned");
  hipError_t e = launch_quantize_append(x_dtype, kv_format, (int)D, K_new, V_new, K_cache, V_cache,
                                        Ks_cache, Vs_cache, rows, n_new, capacity, 0, pos, rows_per_pos,
                                        (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "launch: quantize append kernel");
  return FQKV_OK;
}

int fqkv_quantize_kv_paged(const void* K_new, const void* V_new, int x_dtype, const int32_t* slot_mapping,
                           int64_t tokens, int64_t kv_heads, int64_t D, void* K_pages, void* V_pages,
                           void* Ks_pages, void* Vs_pages, int64_t num_pages, int64_t page_size,
                           int64_t page_stride, int64_t token_stride, int64_t head_stride, int64_t s_page_stride,
                           int64_t s_token_stride, int64_t s_head_stride, int kv_format, void* stream) {
  if (kv_format != FQKV_KV_I8 && kv_format != FQKV_KV_I4 && kv_format != FQKV_KV_FP8)
    return fail(FQKV_ERR_ARG, "kv_format must be FQKV_KV_I8, FQKV_KV_I4 or FQKV_KV_FP8");
  if (x_dtype != FQKV_SRC_F16 && x_dtype != FQKV_SRC_F32 && x_dtype != FQKV_SRC_BF16)
    return fail(FQKV_ERR_ARG, "x_dtype must be FQKV_SRC_F16, FQKV_SRC_F32 or FQKV_SRC_BF16");
  if (D != 64 && D != 128) return fail(FQKV_ERR_ARG, "D: head_dim must be 64 or 128, got %lld", (long long)D);
  if (tokens < 0 || kv_heads < 1)
    return fail(FQKV_ERR_ARG, "shape: tokens must be >= 0 and kv_heads >= 1, got %lld and %lld", (long long)tokens,
                (long long)kv_heads);
  if (num_pages < 1 || page_size < 1 || (page_size & (page_size - 1)) || page_size > (1 << 30) ||
      num_pages > (INT64_MAX >> 31))
    return fail(FQKV_ERR_ARG, "page: num_pages must be in [1, 2^32) and page_size a power of two <= 2^30, got %lld "
                "and %lld", (long long)num_pages, (long long)page_size);
  const int64_t qal = kv_format == FQKV_KV_I4 ? (D == 128 ? 4 : 2) : (D == 128 ? 8 : 4);
  if (page_stride < 0 || token_stride < 0 || head_stride < 0 || page_stride % qal || token_stride % qal ||
      head_stride % qal)
    return fail(FQKV_ERR_ARG, "stride: code strides must be non-negative multiples of %lld bytes", (long long)qal);
  if (s_page_stride < 0 || s_token_stride < 0 || s_head_stride < 0)
    return fail(FQKV_ERR_ARG, "stride: scale strides must be non-negative");
  if (!K_new || !V_new || !slot_mapping || !K_pages || !V_pages || !Ks_pages || !Vs_pages)
    return fail(FQKV_ERR_ARG, "null tensor pointer");
  const uintptr_t xal = (x_dtype != FQKV_SRC_F32 && D == 64) ? 8 : 16;
  if (!aligned(K_new, xal) || !aligned(V_new, xal)) return fail(FQKV_ERR_ARG, "K_new and V_new must be %d-byte aligned", (int)xal);
  if (!aligned(K_pages, (uintptr_t)qal) || !aligned(V_pages, (uintptr_t)qal))
    return fail(FQKV_ERR_ARG, "pages must be %d-byte aligned", (int)qal);
  if (!aligned(Ks_pages, 2) || !aligned(Vs_pages, 2)) return fail(FQKV_ERR_ARG, "scales must be 2-byte aligned");
  if (!aligned(slot_mapping, 4)) return fail(FQKV_ERR_ARG, "slot_mapping must be 4-byte aligned");
  if (tokens == 0) return FQKV_OK;
  const int page_log2 = __builtin_ctzll((unsigned long long)page_size);
  hipError_t e = launch_quantize_pages(x_dtype, kv_format, (int)D, K_new, V_new, slot_mapping, tokens,
                                       kv_heads, K_pages, V_pages, Ks_pages, Vs_pages, num_pages, page_log2,
                                       page_stride, token_stride, head_stride, s_page_stride, s_token_stride,
                                       s_head_stride, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "launch: quantize pages kernel");
  return FQKV_OK;
}

}  // extern "C"
