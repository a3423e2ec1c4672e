/*
 * fqkv_decode.h -- C ABI of the MI355X (gfx950) fused single-query
 * decode-attention library (libfqkv_decode.so).
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer to
 * contiguous memory, every size is a 64-bit integer, `stream` is a
 * hipStream_t passed as void* (NULL = the legacy default stream). All calls
 * are asynchronous on `stream`; none synchronises the device and none
 * allocates device memory (callers pass any workspace; the library's only
 * device state is a static array of split-merge arrival counters).
 *
 * An empty sequence (a paged batch slot with seq_len <= 0) yields zeros.
 *
 * Data formats (the reference's layouts, unchanged):
 *   fp16 KV        K, V: [rows, N, D] __half, row-major
 *   int8 KV        K, V: [rows, N, D] int8, per-token scales Ks, Vs: [rows, N] __half
 *   int4 KV        K, V: [rows, N, D/2] uint8, two values per byte, low nibble
 *                  = even element (byte t holds elements 2t, 2t+1); a nibble n
 *                  decodes as n - 16 when n >= 8; scales as for int8
 *   dequantised value = (float)q * (float)scale, exact in fp32
 *   softmax scale  = 1.0f / sqrtf((float)D); D (head_dim) is 64 or 128
 *
 * Alignment: q, K, V and o_part 16 bytes (K, V 8 bytes for int4 at D = 64);
 * o, scales 2 bytes. Each K or V row block, N rows plus 1040 more, must span
 * at most 4 GiB (fp16 at D = 128: N <= 2^24 - 1040 tokens per KV head).
 *
 * W (and CW) count 64-lane waves per workgroup. W is a maximum: a split too
 * short to give every wave a full pass of 4 16-token tiles runs on fewer
 * waves (at least 2), and the single-block entry points use at most 4 waves
 * once they launch 4 or more workgroups per CU. Results do not depend on W,
 * CW or S beyond fp32 rounding of the merge order.
 *
 * Return value: FQKV_OK (0) on success; otherwise a non-zero FQKV_ERR_* code
 * and fqkv_last_error() describes the failure (thread-local). Argument
 * checks run before any HIP call.
 *
 * Reference interfaces are cited as file:line of
 * emirabayer/Fused-Quantized-KV-Decode-Attention.
 */
#ifndef FQKV_DECODE_H
#define FQKV_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FQKV_OK = 0,
  FQKV_ERR_ARG = 1, /* invalid argument (shape, tuning knob, null pointer, workspace) */
  FQKV_ERR_HIP = 2  /* a HIP runtime call or kernel launch failed */
};

/* KV element formats: fp16 (the reference's), int8 and packed int4 codes with
 * fp16 per-token scales (the reference's quantized formats), bf16 (accepted by
 * the strided and paged entry points, for caches kept in a bf16 model's own
 * dtype) and OCP fp8 e4m3 codes with fp16 per-token scales (accepted wherever
 * int8 is; value = code * scale). bf16 and fp8 have no counterpart in the
 * reference. */
enum { FQKV_KV_F16 = 0, FQKV_KV_I8 = 1, FQKV_KV_I4 = 2, FQKV_KV_BF16 = 3, FQKV_KV_FP8 = 4 };

/* The split merge a call used (fqkv_last_merge_protocol): none (one split),
 * the two-kernel form, the one-kernel form at device scope, or the one-kernel
 * form meeting in one XCD's L2. */
enum { FQKV_MERGE_NONE = 0, FQKV_MERGE_TWO_KERNEL = 1, FQKV_MERGE_DEVICE = 2, FQKV_MERGE_XCD_LOCAL = 3 };

/* element type of a quantizer input; bf16 rows widen exactly to fp32 and are
 * quantized as fp32 (no counterpart in the reference, whose quantizers see
 * fp16 or fp32 tensors) */
enum { FQKV_SRC_F16 = 0, FQKV_SRC_F32 = 1, FQKV_SRC_BF16 = 2 };

/* Message for the last failing call on this thread ("" if none). */
const char* fqkv_last_error(void);

/* Library version string. */
const char* fqkv_version(void);

/*
 * Workspace (bytes) the single-block entry points below use to split a long
 * sequence across workgroups when `rows` alone cannot fill the GPU:
 * rows = batch*kv_heads, G = query heads per KV head (1 for MHA), kv_format
 * FQKV_KV_*, W the waves-per-workgroup knob. Returns 0 when no split is used.
 * A smaller (or NULL) workspace is legal: the entry point then uses as many
 * splits as fit, down to none. Queries the current device's CU count.
 */
size_t fqkv_workspace_bytes(int64_t rows, int64_t G, int64_t N, int64_t D, int kv_format,
                            int64_t W);

/*
 * fp16 MHA decode: o[b] = fp16(softmax(q[b] . K[b]^T / sqrt(D)) V[b]).
 * q: [B, D] fp16, K, V: [B, N, D] fp16, o: [B, D] fp16. W in {2, 4, 8}.
 * Replaces decode_attn_fp16_mw(q, K, V, W) (kernels/decode_attn_fp16_mw.cu:50-63).
 */
int fqkv_decode_attn_fp16_mw(const void* q, const void* K, const void* V, void* o, int64_t B,
                             int64_t N, int64_t D, int64_t W, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * int8-KV MHA decode with per-token fp16 scales.
 * q: [B, D] fp16, K, V: [B, N, D] int8, Ks, Vs: [B, N] fp16, o: [B, D] fp16.
 * Replaces decode_attn_int8_mw(q, K, V, Ks, Vs, W) (kernels/decode_attn_int8_mw.cu:52-64).
 */
int fqkv_decode_attn_int8_mw(const void* q, const void* K, const void* V, const void* Ks,
                             const void* Vs, void* o, int64_t B, int64_t N, int64_t D,
                             int64_t W, void* workspace, size_t workspace_bytes, void* stream);

/*
 * int4-KV MHA decode (packed, low nibble first) with per-token fp16 scales.
 * q: [B, D] fp16, K, V: [B, N, D/2] uint8, Ks, Vs: [B, N] fp16, o: [B, D] fp16.
 * D is the unpacked head_dim (64 or 128; the reference supports 64 only).
 * Replaces decode_attn_int4(q, K, V, Ks, Vs, W) (kernels/decode_attn_int4.cu:47-57).
 */
int fqkv_decode_attn_int4(const void* q, const void* K, const void* V, const void* Ks,
                          const void* Vs, void* o, int64_t B, int64_t N, int64_t D, int64_t W,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * GQA-aware fp16 decode: query head h of batch b reads KV head h / (Hq/Hkv).
 * q: [B, Hq, D], K, V: [B, Hkv, N, D], o: [B, Hq, D], all fp16; Hq % Hkv == 0.
 * Replaces decode_attn_gqa(q, K, V, W) (kernels/decode_attn_gqa.cu:56-68).
 */
int fqkv_decode_attn_gqa(const void* q, const void* K, const void* V, void* o, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int64_t W,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * GQA split-K fp16 decode (partial kernel + combine kernel).
 * q: [Hq, D] fp16, K, V: [Hkv, N, D] fp16, caller-owned fp32 scratch
 * m_part, l_part: [Hq, S], o_part: [Hq, S, D], output o: [Hq, D] fp16.
 * Split s covers tokens [s*c, min(s*c + c, N)) with c = ceil(N/S). Every
 * scratch entry is written: m_part = max score (natural-log units, i.e.
 * scaled by 1/sqrt(D)), l_part = sum exp(score - m), o_part = unnormalised
 * sum exp(score - m) V; an empty split stores (-inf, 0, 0).
 * A batch folds into the head axis: q [B*Hq, D], K [B*Hkv, N, D].
 * W in {2, 4, 8} waves per partial workgroup, CW in {4, 8} combine waves.
 * With S = 1 the partial kernel writes the output as well (one launch).
 * Replaces gqa_sk_fast(q, K, V, m_part, l_part, o_part, o, S, W, CW)
 * (kernels/decode_attn_gqa_sk_fast.cu:95-112).
 */
int fqkv_gqa_sk_fast(const void* q, const void* K, const void* V, float* m_part, float* l_part,
                     float* o_part, void* o, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                     int64_t S, int64_t W, int64_t CW, void* stream);

/*
 * fqkv_gqa_sk_fast without the caller's scratch: the same call, except that
 * the fp32 split partials live in a file-scope device array of the library
 * (8 MiB per device, held until the process ends) instead of caller-owned
 * m_part / l_part / o_part, so a call allocates nothing -- for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The partials need
 * (2 * Hq * S rounded up to a multiple of 4 + Hq * S * D) * 4 bytes; a
 * larger Hq * S is rejected (FQKV_ERR_ARG, message starting "S:") before
 * any HIP call. Every call on a device shares that device's array and leaves
 * its partials there; calls that overlap on one device (other streams, or a
 * captured graph replayed beside them) race on it, so such calls must be
 * ordered. Output, layouts and S / W / CW as for fqkv_gqa_sk_fast, and the
 * result equals it bit for bit. No counterpart in the reference.
 */
int fqkv_gqa_sk_fast_noalloc(const void* q, const void* K, const void* V, void* o, int64_t Hq, int64_t Hkv,
                             int64_t N, int64_t D, int64_t S, int64_t W, int64_t CW, void* stream);

/*
 * GQA-aware decode over an int8, int4 or fp8 e4m3 KV cache (kv_format
 * FQKV_KV_I8 / FQKV_KV_I4 / FQKV_KV_FP8, fp8 laid out as int8) with per-token fp16 scales: the GQA head mapping of
 * fqkv_decode_attn_gqa with the KV format of fqkv_decode_attn_int8_mw /
 * fqkv_decode_attn_int4. q: [B, Hq, D] fp16; K, V: [B, Hkv, N, D] int8 or
 * [B, Hkv, N, D/2] uint8; Ks, Vs: [B, Hkv, N] fp16; o: [B, Hq, D] fp16.
 * No counterpart in the reference, whose int8/int4 kernels are MHA only
 * (decode_attn_int8_mw.cu:52-64, decode_attn_int4.cu:47-57) and whose GQA
 * kernel is fp16 only (decode_attn_gqa.cu:56-68).
 */
int fqkv_decode_attn_gqa_quant(const void* q, const void* K, const void* V, const void* Ks,
                               const void* Vs, void* o, int64_t B, int64_t Hq, int64_t Hkv, int64_t N,
                               int64_t D, int kv_format, int64_t W, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * GQA split-K decode over an int8, int4 or fp8 KV cache: fqkv_gqa_sk_fast with K,
 * V in the quantized layout above and per-token scales Ks, Vs [Hkv, N] fp16
 * (batch folded into the head axis as for fqkv_gqa_sk_fast). Same scratch
 * layout and semantics. No counterpart in the reference (its split-K path,
 * decode_attn_gqa_sk_fast.cu:95-112, is fp16 only). kv_format FQKV_KV_BF16
 * takes bf16 K, V [Hkv, N, D] instead (Ks, Vs ignored).
 */
int fqkv_gqa_sk_fast_quant(const void* q, const void* K, const void* V, const void* Ks, const void* Vs,
                           float* m_part, float* l_part, float* o_part, void* o, int64_t Hq,
                           int64_t Hkv, int64_t N, int64_t D, int kv_format, int64_t S, int64_t W,
                           int64_t CW, void* stream);

/*
 * GQA-aware decode over a KV cache in any strided layout (fp16, bf16, int8
 * or int4 per kv_format): KV head h of sequence b starts at
 * K + b*kv_batch_stride + h*kv_head_stride and its tokens lie kv_token_stride
 * bytes apart (each token row is D fp16 or bf16 / D int8 / D/2 packed bytes);
 * scales likewise in fp16 elements (ignored for fp16 and bf16). [B, Hkv, N, D] is the
 * reference layout; [B, N, Hkv, D] (FlashInfer's NHD, flashinfer_looptimed.py:63-65)
 * has kv_token_stride = Hkv*row_bytes, kv_head_stride = row_bytes,
 * kv_batch_stride = N*Hkv*row_bytes. q [B, Hq, D], o [B, Hq, D] fp16.
 * Strides are multiples of 16 bytes (8 for int4 at D = 64); (N + 1040) *
 * kv_token_stride <= 4 GiB. No counterpart in the reference (contiguous [B, Hkv, N, D] only).
 */
int fqkv_decode_attn_gqa_strided(const void* q, const void* K, const void* V, const void* Ks, const void* Vs,
                                 void* o, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int kv_format,
                                 int64_t kv_batch_stride, int64_t kv_head_stride, int64_t kv_token_stride,
                                 int64_t sc_batch_stride, int64_t sc_head_stride, int64_t sc_token_stride,
                                 int64_t W, void* workspace, size_t workspace_bytes, void* stream);

/*
 * GQA-aware decode over a paged KV cache. Sequence b has seq_lens[b] tokens
 * (int32, device); its token t lives in page page_table[b*max_pages + t/page_size]
 * (int32, device) at in-page position t % page_size. Within page pg, KV head h
 * starts at K_pages + pg*kv_page_stride + h*kv_head_stride, tokens
 * kv_token_stride bytes apart (NHD pages [num_pages, page_size, Hkv, D] and
 * HND pages [num_pages, Hkv, page_size, D] are both strides; any kv_format);
 * scales alike in elements. page_size: a power of two >= 16. max_seq_len bounds every
 * seq_lens[b] (longer sequences are cut there; the kernel also never reads past
 * max_pages pages); a page id outside [0, num_pages) contributes nothing.
 * No counterpart in the reference.
 */
int fqkv_decode_attn_gqa_paged(const void* q, const void* K_pages, const void* V_pages, const void* Ks_pages,
                               const void* Vs_pages, const int32_t* page_table, const int32_t* seq_lens, void* o,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t num_pages, int64_t max_pages,
                               int64_t page_size, int64_t max_seq_len, int64_t D, int kv_format,
                               int64_t kv_page_stride, int64_t kv_head_stride, int64_t kv_token_stride,
                               int64_t sc_page_stride, int64_t sc_head_stride, int64_t sc_token_stride,
                               int64_t W, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Same as fqkv_gqa_sk_fast, additionally recording the hipEvent_t handles
 * ev_begin / ev_end on `stream` immediately before and after the partial
 * kernel, so a caller can time that kernel alone. Either event may be NULL.
 * Instrumented form of decode_attn_gqa_sk_fast.cu:95-112 (no counterpart call).
 */
int fqkv_gqa_sk_fast_timed(const void* q, const void* K, const void* V, float* m_part,
                           float* l_part, float* o_part, void* o, int64_t Hq, int64_t Hkv,
                           int64_t N, int64_t D, int64_t S, int64_t W, int64_t CW, void* stream,
                           void* ev_begin, void* ev_end);

/*
 * Measurement helper: read `bytes` (a multiple of 16) from `src` with
 * 16-byte streaming loads on `blocks` workgroups of 256 threads and write
 * nothing unless `sink` (optional, `blocks` words) receives an impossible
 * checksum. A plain read of the bytes a decode call streams is the
 * ceiling that call can approach; bench.py reports it beside the headline.
 * No counterpart in the reference.
 */
int fqkv_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, void* stream);

/*
 * Hardware check: what gfx950's raw buffer loads return past a descriptor's
 * end. A descriptor over the first `records` bytes (a multiple of 16) of
 * `buf` (`bytes` >= records + 64 long, so no access leaves it) is read at
 * offsets past its end carried in the VGPR offset, the SGPR offset and the
 * immediate field, and with a 16-byte load straddling the end; the nine
 * dwords read go to `out` (see probe_kernels.hip for the order). The attention
 * kernels rely on zeros in those cases. No counterpart in the reference.
 */
int fqkv_probe_buffer_range(const void* buf, size_t bytes, int records, uint32_t* out, void* stream);

/*
 * Dequantise an int8 or int4 KV tensor with the exact device conversion the
 * attention kernels use, writing out[t, d] = (float)q[t, d] * (float)scale[t]
 * for tokens = rows*N token rows. path 0 = the K-side conversion (int -> fp16
 * matrix-core operand), path 1 = the V-side conversion (int -> fp32).
 * Format check for tests/golden bit-exactness; mirrors the kernels' dequant at
 * decode_attn_int8_mw.cu:24,31 and decode_attn_int4.cu:21-23,29-31.
 */
int fqkv_dequant_kv(const void* Kq, const void* Ks, float* out, int64_t tokens, int64_t D,
                    int kv_format, int path, void* stream);

/*
 * Per-token symmetric KV quantizer on the GPU, the producer of the int8 / int4
 * formats above: X [tokens, D] fp16 (x_dtype FQKV_SRC_F16) or fp32
 * (FQKV_SRC_F32) -> Q [tokens, D] int8 (kv_format FQKV_KV_I8, scale =
 * max|x|/127) or [tokens, D/2] uint8 packed low nibble first (FQKV_KV_I4,
 * scale = max|x|/7), scales [tokens] fp16. Bytes identical to the reference's
 * PyTorch expressions evaluated in X's dtype: round-half-even, clamp to
 * [-qmax, qmax], scale clamped to >= 1e-8 (tests/test_kernels.py:32-34,
 * nb:292-299). Alignment: X 16 bytes (8 for fp16 at D = 64), Q 8 / 4 / 2 bytes
 * (int8 D 128 / int8 D 64 or int4 D 128 / int4 D 64), scales 2 bytes.
 * Replaces the PyTorch quantizers qpt (tests/test_kernels.py:32-34) and
 * quant_int4_per_token (nb:292-299), which run on the CPU in the reference.
 * kv_format FQKV_KV_FP8 (no counterpart in the reference) writes fp8 e4m3
 * codes [tokens, D] instead, in fp32 for every source type: s = max(max|x| *
 * fp32(1/448), 1e-8), code = e4m3 round-to-nearest-even of clamp(x / s,
 * +-448), an exact zero as +0, scale fp16(s). bf16 sources (FQKV_SRC_BF16)
 * follow the fp32 expressions for every format.
 */
int fqkv_quantize_kv(const void* X, int x_dtype, void* Q, void* scales, int64_t tokens, int64_t D,
                     int kv_format, void* stream);

/*
 * The quantizer above in append form, for a live decode cache: the new keys
 * and values K_new, V_new [rows, n_new, D] (fp16 or fp32, contiguous) are
 * quantized in one launch into token positions pos .. pos + n_new - 1 of the
 * caches K_cache, V_cache [rows, capacity, D] int8 (or [.., D/2] packed
 * uint8) with scales Ks_cache, Vs_cache [rows, capacity] fp16, all
 * contiguous; rows = batch * kv_heads. The bytes equal fqkv_quantize_kv's on
 * the same tokens; nothing else in the caches changes. No counterpart in the
 * reference (its quantizers run on the CPU over whole tensors,
 * tests/test_kernels.py:32-34, nb:292-299).
 */
int fqkv_quantize_kv_append(const void* K_new, const void* V_new, int x_dtype, void* K_cache, void* V_cache,
                            void* Ks_cache, void* Vs_cache, int64_t rows, int64_t n_new, int64_t capacity,
                            int64_t pos, int64_t D, int kv_format, void* stream);

/*
 * fqkv_quantize_kv_append with the positions on the device: the new tokens of
 * cache row r go to positions pos[r / rows_per_pos] .. + n_new - 1, read by the
 * kernel (pos: int32, rows / rows_per_pos entries, e.g. one per sequence with
 * rows_per_pos = KV heads), so a captured graph appends wherever the cache
 * ends at replay time. Rows whose tokens would leave [0, capacity) are not
 * written. No counterpart in the reference; for decode loops replayed from
 * HIP graphs over a preallocated int8 / int4 cache.
 */
int fqkv_quantize_kv_append_at(const void* K_new, const void* V_new, int x_dtype, void* K_cache, void* V_cache,
                               void* Ks_cache, void* Vs_cache, int64_t rows, int64_t n_new, int64_t capacity,
                               const int32_t* pos, int64_t rows_per_pos, int64_t D, int kv_format, void* stream);

/*
 * The quantizer writing into a paged int8 / int4 cache, as serving engines
 * fill one: token t of K_new, V_new [tokens, kv_heads, D] (fp16 or fp32,
 * contiguous) goes to slot slot_mapping[t] = page * page_size + offset (int32,
 * device memory) of the pages the paged decode entry point reads. Codes of
 * KV head h of a slot sit at page * page_stride + offset * token_stride +
 * h * head_stride bytes from K_pages / V_pages (multiples of 8 / 4 / 4 / 2
 * bytes for int8 D 128 / int8 D 64 / int4 D 128 / int4 D 64), its scale at
 * the same position in elements by the s_* strides, so token-major (NHD) and
 * head-major (HND) pages are both served. A slot outside
 * [0, num_pages * page_size), e.g. -1 for a padding token, writes nothing.
 * Bytes equal fqkv_quantize_kv's on the same rows. No counterpart in the
 * reference (its caches are contiguous fp16 / int8 / int4 tensors quantized
 * on the host); for serving callers of fqkv_decode_attn_gqa_paged.
 */
int fqkv_quantize_kv_paged(const void* K_new, const void* V_new, int x_dtype, const int32_t* slot_mapping,
                           int64_t tokens, int64_t kv_heads, int64_t D, void* K_pages, void* V_pages,
                           void* Ks_pages, void* Vs_pages, int64_t num_pages, int64_t page_size,
                           int64_t page_stride, int64_t token_stride, int64_t head_stride, int64_t s_page_stride,
                           int64_t s_token_stride, int64_t s_head_stride, int kv_format, void* stream);

/*
 * Split merge mode for calls that split the sequence (gqa_sk_fast with S > 1
 * and the internal splits of the single-block entry points). Default (0):
 * one kernel per call; the last workgroup of each head group to finish merges
 * that group's split partials, using library-owned arrival counters. The
 * counters come in 128 slots per device: each stream keeps one of 12 slots for
 * its eager calls (first come, first served), and each stream of each stream
 * capture (streams that join a capture through event waits each count) takes
 * one of the other 116 for the graph it records; calls on a stream or capture
 * with no free slot, and calls on hipStreamPerThread, use the two-kernel
 * merge (fqkv_merge_fallback_count counts the calls that found no free slot).
 * So calls that may overlap never share a slot, with two exceptions a caller
 * must avoid: replaying one captured graph on two streams at once (those
 * replays also share the caller's scratch and output), and destroying a
 * stream with split calls still queued and creating a new one that gets the
 * same handle before they finish. Capture slots stay taken until
 * fqkv_release_capture_slots. 1: a partial kernel then a separate combine
 * kernel, as the reference launches them (decode_attn_gqa_sk_fast.cu:100-111).
 * Results agree to fp32 rounding. Process-wide; returns FQKV_OK.
 *
 * The first eager split call on a device (not one on a capturing stream)
 * launches a small probe on its stream and waits for it, once per process
 * and device: it records which XCD runs each workgroup. When every split of a
 * head group runs on one XCD (16 or more splits, head groups a multiple of
 * the XCD count) and the stream has no CU mask that leaves CUs out, the
 * one-kernel merge keeps its partials and counters in that XCD's L2 instead
 * of device-scope memory; results are bit for bit the same.
 * FQKV_XCD_LOCAL_MERGE=0 in the environment skips the probe and keeps the
 * device-scope protocol.
 */
int fqkv_set_two_kernel_merge(int enable);

/*
 * Diagnostics of the split merge (no counterpart in the reference; for tests,
 * benchmarks and callers checking which path their calls take).
 * fqkv_last_merge_protocol: the FQKV_MERGE_* protocol of the calling thread's
 * last successful decode call. fqkv_merge_fallback_count: calls since the
 * library loaded that took the two-kernel merge because every counter slot of
 * their kind (eager or captured) was taken. fqkv_xcd_period: the XCD period
 * the probe found on `device` (> 0), 0 while it has not run, -1 when it found
 * no usable order (or FQKV_XCD_LOCAL_MERGE=0).
 */
int fqkv_last_merge_protocol(void);
int64_t fqkv_merge_fallback_count(void);
int fqkv_xcd_period(int device);

/*
 * Frees every capture slot of the current device, so later captures take
 * the one-kernel merge again once all 116 have been used. Call it only after
 * destroying every graph that captured split calls on this device: a graph
 * replayed afterwards could share its counters with a new capture's. No
 * counterpart in the reference. Returns FQKV_OK.
 */
int fqkv_release_capture_slots(void);

/*
 * Measurement knob: with `enable` nonzero, fp16 calls at D = 128 whose work
 * items hold 1 or 4 query heads (MHA, and GQA with 4 query heads per KV
 * head) on contiguous rows compute P.V on the vector ALUs instead of the
 * matrix cores; everything else in the kernel is unchanged, so timing the
 * two settings compares the two products. Other calls are not affected.
 * Process-wide, not synchronised with calls in flight. No counterpart in
 * the reference. Returns FQKV_OK.
 */
int fqkv_set_pv_valu(int enable);

/* Number of compute units of the current device (used by the split heuristic). */
int fqkv_device_cu_count(int* cu_count);

/*
 * Splits the single-block entry points use for a problem (1 = no split), as
 * chosen from the current device's CU count; exposed for tests and tooling.
 */
int64_t fqkv_choose_splits(int64_t rows, int64_t G, int64_t N, int64_t D, int kv_format,
                           int64_t W);

#ifdef __cplusplus
}
#endif

#endif /* FQKV_DECODE_H */
