// PyTorch binding of libfqkv_decode: the reference's extension call surface.
//
// Five functions with the reference's names, argument order, tensor layouts
// and return conventions (kernels/decode_attn_fp16_mw.cu:50,64;
// decode_attn_int8_mw.cu:52,65; decode_attn_int4.cu:47,58;
// decode_attn_gqa.cu:56,69; decode_attn_gqa_sk_fast.cu:95,113). Validation
// is a superset of the reference's TORCH_CHECKs: each message starts with
// the reference's keyword ("cuda", "fp16", "contig", "D", "W", "int8",
// "packed uint8", "CW", "partial", "combine", "launch"). Work is launched on
// PyTorch's current HIP stream of the inputs' device (the reference used
// the legacy default stream), so HIP graph capture and stream overlap work.
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "fqkv_decode.h"

namespace {

void check_rc(int rc, const char* tag) {
  TORCH_CHECK(rc == FQKV_OK, tag, ": ", fqkv_last_error());
}

void* cur_stream(const torch::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

void check_gpu(std::initializer_list<const torch::Tensor*> ts) {
  const torch::Tensor& first = **ts.begin();
  for (const torch::Tensor* t : ts) {
    TORCH_CHECK(t->is_cuda(), "cuda: all tensors must be on the GPU");
    TORCH_CHECK(t->device() == first.device(), "cuda: all tensors must be on the same device");
    TORCH_CHECK(t->is_contiguous(), "contig: all tensors must be contiguous");
  }
}

// Device checks for tensors that may be strided views (paged caches).
void check_gpu_strided(std::initializer_list<const torch::Tensor*> ts, const torch::Tensor& like) {
  for (const torch::Tensor* t : ts) {
    TORCH_CHECK(t->is_cuda(), "cuda: all tensors must be on the GPU");
    TORCH_CHECK(t->device() == like.device(), "cuda: all tensors must be on the same device");
  }
}

void check_half(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == torch::kHalf, "fp16: ", name, " must be float16");
}

void check_W(int64_t W) { TORCH_CHECK(W == 2 || W == 4 || W == 8, "W: must be 2, 4 or 8, got ", W); }

void check_D(int64_t D) { TORCH_CHECK(D == 64 || D == 128, "D: head_dim must be 64 or 128, got ", D); }

// KV code format of a quantized cache tensor's dtype (FQKV_KV_I8 / _I4 / _FP8), -1 for any other.
int code_format(const torch::Tensor& C) {
  switch (C.scalar_type()) {
    case torch::kChar: return FQKV_KV_I8;
    case torch::kByte: return FQKV_KV_I4;
    case torch::kFloat8_e4m3fn: return FQKV_KV_FP8;
    default: return -1;
  }
}

// Quantizer source element type (FQKV_SRC_*), -1 for any other dtype.
int src_of(const torch::Tensor& X) {
  switch (X.scalar_type()) {
    case torch::kHalf: return FQKV_SRC_F16;
    case torch::kFloat: return FQKV_SRC_F32;
    case torch::kBFloat16: return FQKV_SRC_BF16;
    default: return -1;
  }
}

torch::Tensor workspace_for(const torch::Tensor& q, int64_t rows, int64_t G, int64_t N, int64_t D,
                            int fmt, int64_t W) {
  const c10::DeviceGuard guard(q.device());
  const size_t bytes = fqkv_workspace_bytes(rows, G, N, D, fmt, W);
  if (bytes == 0) return torch::Tensor();
  return torch::empty({(int64_t)bytes}, q.options().dtype(torch::kUInt8));
}

// decode_attn_fp16_mw(q[B,D], K[B,N,D], V[B,N,D], W) -> o[B,D]
torch::Tensor decode_attn_fp16_mw(torch::Tensor q, torch::Tensor K, torch::Tensor V, int64_t W) {
  check_gpu({&q, &K, &V});
  check_half(q, "q");
  check_half(K, "K");
  check_half(V, "V");
  TORCH_CHECK(q.dim() == 2 && K.dim() == 3 && V.sizes() == K.sizes() && q.size(0) == K.size(0) &&
                  q.size(1) == K.size(2),
              "shape: expected q [B,D], K and V [B,N,D]; got q ", q.sizes(), ", K ", K.sizes(), ", V ", V.sizes());
  const int64_t B = K.size(0), N = K.size(1), D = K.size(2);
  check_D(D);
  check_W(W);
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  const c10::DeviceGuard guard(q.device());
  auto o = torch::empty({B, D}, q.options());
  auto ws = workspace_for(q, B, 1, N, D, FQKV_KV_F16, W);
  check_rc(fqkv_decode_attn_fp16_mw(q.data_ptr(), K.data_ptr(), V.data_ptr(), o.data_ptr(), B, N, D, W,
                                    ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? ws.numel() : 0,
                                    cur_stream(q)),
           "launch");
  return o;
}

torch::Tensor quant_common(int fmt, torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                           torch::Tensor Vs, int64_t W) {
  check_gpu({&q, &K, &V, &Ks, &Vs});
  check_half(q, "q");
  check_half(Ks, "Ks");
  check_half(Vs, "Vs");
  if (fmt == FQKV_KV_I8) {
    TORCH_CHECK(K.scalar_type() == torch::kChar && V.scalar_type() == torch::kChar, "int8: K and V must be int8");
  } else {
    TORCH_CHECK(K.scalar_type() == torch::kByte && V.scalar_type() == torch::kByte,
                "packed uint8: K and V must be uint8 holding two int4 values per byte");
  }
  TORCH_CHECK(q.dim() == 2 && K.dim() == 3 && V.sizes() == K.sizes() && q.size(0) == K.size(0),
              "shape: expected q [B,D], K and V [B,N,", fmt == FQKV_KV_I4 ? "D/2" : "D", "]; got q ", q.sizes(),
              ", K ", K.sizes(), ", V ", V.sizes());
  const int64_t B = K.size(0), N = K.size(1);
  const int64_t D = fmt == FQKV_KV_I8 ? K.size(2) : 2 * K.size(2);
  if (fmt == FQKV_KV_I4) {
    TORCH_CHECK(D == 64 || D == 128, "D: packed int4 rows must hold 32 or 64 bytes (head_dim 64 or 128), got ",
                K.size(2), " bytes");
  }
  check_D(D);
  TORCH_CHECK(q.size(1) == D, "shape: q head_dim ", q.size(1), " does not match KV head_dim ", D);
  TORCH_CHECK(Ks.dim() == 2 && Ks.size(0) == B && Ks.size(1) == N && Vs.sizes() == Ks.sizes(),
              "shape: expected per-token scales Ks and Vs [B,N]; got ", Ks.sizes(), " and ", Vs.sizes());
  check_W(W);
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  const c10::DeviceGuard guard(q.device());
  auto o = torch::empty({B, D}, q.options());
  auto ws = workspace_for(q, B, 1, N, D, fmt, W);
  void* wsp = ws.defined() ? ws.data_ptr() : nullptr;
  const size_t wsb = ws.defined() ? ws.numel() : 0;
  const int rc = fmt == FQKV_KV_I8
                     ? fqkv_decode_attn_int8_mw(q.data_ptr(), K.data_ptr(), V.data_ptr(), Ks.data_ptr(),
                                                Vs.data_ptr(), o.data_ptr(), B, N, D, W, wsp, wsb, cur_stream(q))
                     : fqkv_decode_attn_int4(q.data_ptr(), K.data_ptr(), V.data_ptr(), Ks.data_ptr(),
                                             Vs.data_ptr(), o.data_ptr(), B, N, D, W, wsp, wsb, cur_stream(q));
  check_rc(rc, "launch");
  return o;
}

// decode_attn_int8_mw(q[B,D], K[B,N,D] int8, V, Ks[B,N] fp16, Vs, W) -> o[B,D]
torch::Tensor decode_attn_int8_mw(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                                  torch::Tensor Vs, int64_t W) {
  return quant_common(FQKV_KV_I8, q, K, V, Ks, Vs, W);
}

// decode_attn_int4(q[B,D], K[B,N,D/2] uint8, V, Ks[B,N] fp16, Vs, W) -> o[B,D]
torch::Tensor decode_attn_int4(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                               torch::Tensor Vs, int64_t W) {
  return quant_common(FQKV_KV_I4, q, K, V, Ks, Vs, W);
}

// decode_attn_gqa(q[B,Hq,D], K[B,Hkv,N,D], V, W) -> o[B,Hq,D]
torch::Tensor decode_attn_gqa(torch::Tensor q, torch::Tensor K, torch::Tensor V, int64_t W) {
  check_gpu({&q, &K, &V});
  check_half(q, "q");
  check_half(K, "K");
  check_half(V, "V");
  TORCH_CHECK(q.dim() == 3 && K.dim() == 4 && V.sizes() == K.sizes() && q.size(0) == K.size(0) &&
                  q.size(2) == K.size(3),
              "shape: expected q [B,Hq,D], K and V [B,Hkv,N,D]; got q ", q.sizes(), ", K ", K.sizes(), ", V ",
              V.sizes());
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(2), Hkv = K.size(1), N = K.size(2);
  check_D(D);
  check_W(W);
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "heads: Hq (", Hq, ") must be a multiple of Hkv (", Hkv, ")");
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  const c10::DeviceGuard guard(q.device());
  auto o = torch::empty({B, Hq, D}, q.options());
  auto ws = workspace_for(q, B * Hkv, Hq / Hkv, N, D, FQKV_KV_F16, W);
  check_rc(fqkv_decode_attn_gqa(q.data_ptr(), K.data_ptr(), V.data_ptr(), o.data_ptr(), B, Hq, Hkv, N, D, W,
                                ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? ws.numel() : 0,
                                cur_stream(q)),
           "launch");
  return o;
}

void sk_checks(const torch::Tensor& q, const torch::Tensor& K, const torch::Tensor& V, const torch::Tensor& m_part,
               const torch::Tensor& l_part, const torch::Tensor& o_part, const torch::Tensor& o, int64_t S,
               int64_t W, int64_t CW) {
  check_gpu({&q, &K, &V, &m_part, &l_part, &o_part, &o});
  check_half(q, "q");
  check_half(K, "K");
  check_half(V, "V");
  check_half(o, "o");
  TORCH_CHECK(m_part.scalar_type() == torch::kFloat && l_part.scalar_type() == torch::kFloat &&
                  o_part.scalar_type() == torch::kFloat,
              "partial: m_part, l_part and o_part must be float32");
  TORCH_CHECK(q.dim() == 2 && K.dim() == 3 && V.sizes() == K.sizes() && q.size(1) == K.size(2),
              "shape: expected q [Hq,D], K and V [Hkv,N,D]; got q ", q.sizes(), ", K ", K.sizes(), ", V ",
              V.sizes());
  const int64_t Hq = q.size(0), D = q.size(1), Hkv = K.size(0), N = K.size(1);
  check_D(D);
  check_W(W);
  TORCH_CHECK(CW == 4 || CW == 8, "CW: must be 4 or 8, got ", CW);
  TORCH_CHECK(S >= 1, "S: split count must be >= 1, got ", S);
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "heads: Hq (", Hq, ") must be a multiple of Hkv (", Hkv, ")");
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  TORCH_CHECK(m_part.numel() == Hq * S && l_part.numel() == Hq * S,
              "partial: m_part and l_part must hold Hq*S = ", Hq * S, " floats");
  TORCH_CHECK(o_part.numel() == Hq * S * D, "partial: o_part must hold Hq*S*D = ", Hq * S * D, " floats");
  TORCH_CHECK(o.numel() == Hq * D, "combine: o must hold Hq*D = ", Hq * D, " halves");
}

// gqa_sk_fast_bf16: gqa_sk_fast over bf16 K and V [Hkv,N,D] (q, o fp16), the same scratch; no
// counterpart in the reference (its split-K is fp16 only).
void gqa_sk_fast_bf16(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor m_part, torch::Tensor l_part,
                      torch::Tensor o_part, torch::Tensor o, int64_t S, int64_t W, int64_t CW) {
  TORCH_CHECK(K.scalar_type() == torch::kBFloat16 && V.scalar_type() == torch::kBFloat16,
              "bf16: K and V must be bfloat16");
  // the fp16 checks with K and V standing in as fp16 views of the same shape
  sk_checks(q, K.view(torch::kHalf), V.view(torch::kHalf), m_part, l_part, o_part, o, S, W, CW);
  const c10::DeviceGuard guard(q.device());
  check_rc(fqkv_gqa_sk_fast_quant(q.data_ptr(), K.data_ptr(), V.data_ptr(), nullptr, nullptr,
                                  m_part.data_ptr<float>(), l_part.data_ptr<float>(), o_part.data_ptr<float>(),
                                  o.data_ptr(), q.size(0), K.size(0), K.size(1), q.size(1), FQKV_KV_BF16, S, W, CW,
                                  cur_stream(q)),
           "launch");
}

// gqa_sk_fast(q[Hq,D], K[Hkv,N,D], V, m_part[Hq,S], l_part[Hq,S], o_part[Hq,S,D], o[Hq,D], S, W, CW)
void gqa_sk_fast(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor m_part, torch::Tensor l_part,
                 torch::Tensor o_part, torch::Tensor o, int64_t S, int64_t W, int64_t CW) {
  sk_checks(q, K, V, m_part, l_part, o_part, o, S, W, CW);
  const c10::DeviceGuard guard(q.device());
  check_rc(fqkv_gqa_sk_fast(q.data_ptr(), K.data_ptr(), V.data_ptr(), m_part.data_ptr<float>(),
                            l_part.data_ptr<float>(), o_part.data_ptr<float>(), o.data_ptr(), q.size(0), K.size(0),
                            K.size(1), q.size(1), S, W, CW, cur_stream(q)),
           "launch");
}

// gqa_sk_fast plus hipEvent records around the partial kernel (timing only).
void gqa_sk_fast_timed(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor m_part,
                       torch::Tensor l_part, torch::Tensor o_part, torch::Tensor o, int64_t S, int64_t W,
                       int64_t CW, int64_t ev_begin, int64_t ev_end) {
  sk_checks(q, K, V, m_part, l_part, o_part, o, S, W, CW);
  const c10::DeviceGuard guard(q.device());
  check_rc(fqkv_gqa_sk_fast_timed(q.data_ptr(), K.data_ptr(), V.data_ptr(), m_part.data_ptr<float>(),
                                  l_part.data_ptr<float>(), o_part.data_ptr<float>(), o.data_ptr(), q.size(0),
                                  K.size(0), K.size(1), q.size(1), S, W, CW, cur_stream(q), (void*)ev_begin,
                                  (void*)ev_end),
           "launch");
}

// ---- quantized GQA and split-K (no counterpart in the reference) ----

// dtype of an int8 / packed-int4 K, V pair; returns the unpacked head_dim.
int64_t quant_kv_dims(int fmt, const torch::Tensor& K, const torch::Tensor& V) {
  if (fmt == FQKV_KV_I8) {
    TORCH_CHECK(K.scalar_type() == torch::kChar && V.scalar_type() == torch::kChar, "int8: K and V must be int8");
  } else if (fmt == FQKV_KV_FP8) {
    TORCH_CHECK(K.scalar_type() == torch::kFloat8_e4m3fn && V.scalar_type() == torch::kFloat8_e4m3fn,
                "fp8: K and V must be float8_e4m3fn");
  } else {
    TORCH_CHECK(K.scalar_type() == torch::kByte && V.scalar_type() == torch::kByte,
                "packed uint8: K and V must be uint8 holding two int4 values per byte");
  }
  TORCH_CHECK(V.sizes() == K.sizes(), "shape: K and V must have the same shape; got ", K.sizes(), " and ",
              V.sizes());
  const int64_t D = fmt == FQKV_KV_I4 ? 2 * K.size(-1) : K.size(-1);
  check_D(D);
  return D;
}

// decode_attn_gqa_int8 / _int4 (q[B,Hq,D], K[B,Hkv,N,D or D/2], V, Ks[B,Hkv,N] fp16, Vs, W) -> o[B,Hq,D]
torch::Tensor decode_attn_gqa_quant(int fmt, torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                                    torch::Tensor Vs, int64_t W) {
  check_gpu({&q, &K, &V, &Ks, &Vs});
  check_half(q, "q");
  check_half(Ks, "Ks");
  check_half(Vs, "Vs");
  TORCH_CHECK(q.dim() == 3 && K.dim() == 4 && q.size(0) == K.size(0),
              "shape: expected q [B,Hq,D], K and V [B,Hkv,N,", fmt == FQKV_KV_I4 ? "D/2" : "D", "]; got q ",
              q.sizes(), ", K ", K.sizes());
  const int64_t D = quant_kv_dims(fmt, K, V);
  const int64_t B = q.size(0), Hq = q.size(1), Hkv = K.size(1), N = K.size(2);
  TORCH_CHECK(q.size(2) == D, "shape: q head_dim ", q.size(2), " does not match KV head_dim ", D);
  TORCH_CHECK(Ks.dim() == 3 && Ks.size(0) == B && Ks.size(1) == Hkv && Ks.size(2) == N && Vs.sizes() == Ks.sizes(),
              "shape: expected per-token scales Ks and Vs [B,Hkv,N]; got ", Ks.sizes(), " and ", Vs.sizes());
  check_W(W);
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "heads: Hq (", Hq, ") must be a multiple of Hkv (", Hkv, ")");
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  const c10::DeviceGuard guard(q.device());
  auto o = torch::empty({B, Hq, D}, q.options());
  auto ws = workspace_for(q, B * Hkv, Hq / Hkv, N, D, fmt, W);
  check_rc(fqkv_decode_attn_gqa_quant(q.data_ptr(), K.data_ptr(), V.data_ptr(), Ks.data_ptr(), Vs.data_ptr(),
                                      o.data_ptr(), B, Hq, Hkv, N, D, fmt, W,
                                      ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? ws.numel() : 0,
                                      cur_stream(q)),
           "launch");
  return o;
}

torch::Tensor decode_attn_gqa_int8(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                                   torch::Tensor Vs, int64_t W) {
  return decode_attn_gqa_quant(FQKV_KV_I8, q, K, V, Ks, Vs, W);
}
torch::Tensor decode_attn_gqa_int4(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                                   torch::Tensor Vs, int64_t W) {
  return decode_attn_gqa_quant(FQKV_KV_I4, q, K, V, Ks, Vs, W);
}
torch::Tensor decode_attn_gqa_fp8(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                                  torch::Tensor Vs, int64_t W) {
  return decode_attn_gqa_quant(FQKV_KV_FP8, q, K, V, Ks, Vs, W);
}

// gqa_sk_fast_int8 / _int4 (q[Hq,D], K[Hkv,N,D or D/2], V, Ks[Hkv,N], Vs, m_part, l_part, o_part, o, S, W, CW)
void gqa_sk_fast_quant(int fmt, torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks,
                       torch::Tensor Vs, torch::Tensor m_part, torch::Tensor l_part, torch::Tensor o_part,
                       torch::Tensor o, int64_t S, int64_t W, int64_t CW) {
  check_gpu({&q, &K, &V, &Ks, &Vs, &m_part, &l_part, &o_part, &o});
  check_half(q, "q");
  check_half(o, "o");
  check_half(Ks, "Ks");
  check_half(Vs, "Vs");
  TORCH_CHECK(m_part.scalar_type() == torch::kFloat && l_part.scalar_type() == torch::kFloat &&
                  o_part.scalar_type() == torch::kFloat,
              "partial: m_part, l_part and o_part must be float32");
  TORCH_CHECK(q.dim() == 2 && K.dim() == 3, "shape: expected q [Hq,D], K and V [Hkv,N,",
              fmt == FQKV_KV_I4 ? "D/2" : "D", "]; got q ", q.sizes(), ", K ", K.sizes());
  const int64_t D = quant_kv_dims(fmt, K, V);
  const int64_t Hq = q.size(0), Hkv = K.size(0), N = K.size(1);
  TORCH_CHECK(q.size(1) == D, "shape: q head_dim ", q.size(1), " does not match KV head_dim ", D);
  TORCH_CHECK(Ks.dim() == 2 && Ks.size(0) == Hkv && Ks.size(1) == N && Vs.sizes() == Ks.sizes(),
              "shape: expected per-token scales Ks and Vs [Hkv,N]; got ", Ks.sizes(), " and ", Vs.sizes());
  check_W(W);
  TORCH_CHECK(CW == 4 || CW == 8, "CW: must be 4 or 8, got ", CW);
  TORCH_CHECK(S >= 1, "S: split count must be >= 1, got ", S);
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "heads: Hq (", Hq, ") must be a multiple of Hkv (", Hkv, ")");
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  TORCH_CHECK(m_part.numel() == Hq * S && l_part.numel() == Hq * S,
              "partial: m_part and l_part must hold Hq*S = ", Hq * S, " floats");
  TORCH_CHECK(o_part.numel() == Hq * S * D, "partial: o_part must hold Hq*S*D = ", Hq * S * D, " floats");
  TORCH_CHECK(o.numel() == Hq * D, "combine: o must hold Hq*D = ", Hq * D, " halves");
  const c10::DeviceGuard guard(q.device());
  check_rc(fqkv_gqa_sk_fast_quant(q.data_ptr(), K.data_ptr(), V.data_ptr(), Ks.data_ptr(), Vs.data_ptr(),
                                  m_part.data_ptr<float>(), l_part.data_ptr<float>(), o_part.data_ptr<float>(),
                                  o.data_ptr(), Hq, Hkv, N, D, fmt, S, W, CW, cur_stream(q)),
           "launch");
}

void gqa_sk_fast_int8(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks, torch::Tensor Vs,
                      torch::Tensor m_part, torch::Tensor l_part, torch::Tensor o_part, torch::Tensor o, int64_t S,
                      int64_t W, int64_t CW) {
  gqa_sk_fast_quant(FQKV_KV_I8, q, K, V, Ks, Vs, m_part, l_part, o_part, o, S, W, CW);
}
void gqa_sk_fast_int4(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks, torch::Tensor Vs,
                      torch::Tensor m_part, torch::Tensor l_part, torch::Tensor o_part, torch::Tensor o, int64_t S,
                      int64_t W, int64_t CW) {
  gqa_sk_fast_quant(FQKV_KV_I4, q, K, V, Ks, Vs, m_part, l_part, o_part, o, S, W, CW);
}
void gqa_sk_fast_fp8(torch::Tensor q, torch::Tensor K, torch::Tensor V, torch::Tensor Ks, torch::Tensor Vs,
                     torch::Tensor m_part, torch::Tensor l_part, torch::Tensor o_part, torch::Tensor o, int64_t S,
                     int64_t W, int64_t CW) {
  gqa_sk_fast_quant(FQKV_KV_FP8, q, K, V, Ks, Vs, m_part, l_part, o_part, o, S, W, CW);
}

// ---- other KV layouts (no counterpart in the reference) ----

// int8 / int4 codes, which come with per-token scales
bool quant_fmt(int fmt) { return fmt == FQKV_KV_I8 || fmt == FQKV_KV_I4 || fmt == FQKV_KV_FP8; }

// KV format from K's dtype; returns FQKV_KV_*, sets D (unpacked head_dim) and the element size.
int kv_format_of(const torch::Tensor& K, int64_t* D, int64_t* elem) {
  if (K.scalar_type() == torch::kHalf || K.scalar_type() == torch::kBFloat16) {
    *D = K.size(-1);
    *elem = 2;
    return K.scalar_type() == torch::kHalf ? FQKV_KV_F16 : FQKV_KV_BF16;
  }
  if (K.scalar_type() == torch::kChar || K.scalar_type() == torch::kFloat8_e4m3fn) {
    *D = K.size(-1);
    *elem = 1;
    return K.scalar_type() == torch::kChar ? FQKV_KV_I8 : FQKV_KV_FP8;
  }
  TORCH_CHECK(K.scalar_type() == torch::kByte, "fp16: K must be float16, bfloat16, int8 or packed uint8 (int4)");
  *D = 2 * K.size(-1);
  *elem = 1;
  return FQKV_KV_I4;
}

void check_scales(int fmt, const c10::optional<torch::Tensor>& Ks, const c10::optional<torch::Tensor>& Vs,
                  at::IntArrayRef want) {
  if (!quant_fmt(fmt)) return;
  TORCH_CHECK(Ks.has_value() && Vs.has_value(), "int8: int8 / int4 K and V need per-token scales Ks and Vs");
  check_gpu_strided({&*Ks, &*Vs}, *Ks);
  check_half(*Ks, "Ks");
  check_half(*Vs, "Vs");
  TORCH_CHECK(Ks->sizes() == want && Vs->sizes() == want && Ks->strides() == Vs->strides(),
              "shape: scales must be ", want, " with equal strides; got ", Ks->sizes(), " and ", Vs->sizes());
}

// decode_attn_gqa_nhd(q[B,Hq,D], K[B,N,Hkv,D or D/2], V, W, Ks=None[B,N,Hkv], Vs=None) -> o[B,Hq,D]:
// the token-major layout FlashInfer uses (flashinfer_looptimed.py:63-65).
torch::Tensor decode_attn_gqa_nhd(torch::Tensor q, torch::Tensor K, torch::Tensor V, int64_t W,
                                  c10::optional<torch::Tensor> Ks, c10::optional<torch::Tensor> Vs) {
  check_gpu({&q, &K, &V});
  check_half(q, "q");
  TORCH_CHECK(q.dim() == 3 && K.dim() == 4 && V.sizes() == K.sizes() && V.scalar_type() == K.scalar_type() &&
                  q.size(0) == K.size(0),
              "shape: expected q [B,Hq,D], K and V [B,N,Hkv,D]; got q ", q.sizes(), ", K ", K.sizes());
  TORCH_CHECK(K.is_contiguous() && V.is_contiguous(), "contig: K and V must be contiguous [B,N,Hkv,D]");
  int64_t D = 0, elem = 0;
  const int fmt = kv_format_of(K, &D, &elem);
  check_D(D);
  TORCH_CHECK(q.size(2) == D, "shape: q head_dim ", q.size(2), " does not match KV head_dim ", D);
  const int64_t B = q.size(0), Hq = q.size(1), N = K.size(1), Hkv = K.size(2);
  check_W(W);
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "heads: Hq (", Hq, ") must be a multiple of Hkv (", Hkv, ")");
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  check_scales(fmt, Ks, Vs, {B, N, Hkv});
  const bool quant = quant_fmt(fmt);
  if (quant) {
    TORCH_CHECK(Ks->device() == q.device(), "cuda: all tensors must be on the same device");
    TORCH_CHECK(Ks->is_contiguous() && Vs->is_contiguous(), "contig: scales must be contiguous");
  }
  const c10::DeviceGuard guard(q.device());
  auto o = torch::empty({B, Hq, D}, q.options());
  auto ws = workspace_for(q, B * Hkv, Hq / Hkv, N, D, fmt, W);
  const int64_t rb = K.size(3) * elem;
  check_rc(fqkv_decode_attn_gqa_strided(q.data_ptr(), K.data_ptr(), V.data_ptr(),
                                        quant ? Ks->data_ptr() : nullptr, quant ? Vs->data_ptr() : nullptr,
                                        o.data_ptr(), B, Hq, Hkv, N, D,
                                        fmt, N * Hkv * rb, rb, Hkv * rb, N * Hkv, 1, Hkv, W,
                                        ws.defined() ? ws.data_ptr() : nullptr, ws.defined() ? ws.numel() : 0,
                                        cur_stream(q)),
           "launch");
  return o;
}

// decode_attn_gqa_strided(q[B,Hq,D], K[B,Hkv,N,D or D/2], V, W, Ks=None[B,Hkv,N], Vs=None) -> o[B,Hq,D]:
// K and V may be any strided views with contiguous rows (the last dim), e.g. the first N tokens of a
// preallocated [B,Hkv,capacity,D] cache, or a token-major [B,N,Hkv,D] cache passed as transpose(1,2);
// the scales are views of the same kind. The strides must satisfy fqkv_decode_attn_gqa_strided's rules.
torch::Tensor decode_attn_gqa_strided(torch::Tensor q, torch::Tensor K, torch::Tensor V, int64_t W,
                                      c10::optional<torch::Tensor> Ks, c10::optional<torch::Tensor> Vs) {
  check_gpu({&q});
  check_gpu_strided({&K, &V}, q);
  check_half(q, "q");
  TORCH_CHECK(q.dim() == 3 && K.dim() == 4 && V.sizes() == K.sizes() && V.strides() == K.strides() &&
                  V.scalar_type() == K.scalar_type() && q.size(0) == K.size(0),
              "shape: expected q [B,Hq,D], K and V [B,Hkv,N,D] views with equal strides; got q ", q.sizes(),
              ", K ", K.sizes(), " ", K.strides(), ", V ", V.sizes(), " ", V.strides());
  TORCH_CHECK(K.size(3) == 1 || K.stride(3) == 1, "contig: K and V rows (the last dim) must be contiguous");
  int64_t D = 0, elem = 0;
  const int fmt = kv_format_of(K, &D, &elem);
  check_D(D);
  TORCH_CHECK(q.size(2) == D, "shape: q head_dim ", q.size(2), " does not match KV head_dim ", D);
  const int64_t B = q.size(0), Hq = q.size(1), Hkv = K.size(1), N = K.size(2);
  check_W(W);
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "heads: Hq (", Hq, ") must be a multiple of Hkv (", Hkv, ")");
  TORCH_CHECK(N >= 1, "N: need at least one cached token");
  check_scales(fmt, Ks, Vs, {B, Hkv, N});
  const bool quant = quant_fmt(fmt);
  if (quant) TORCH_CHECK(Ks->device() == q.device(), "cuda: all tensors must be on the same device");
  const c10::DeviceGuard guard(q.device());
  auto o = torch::empty({B, Hq, D}, q.options());
  auto ws = workspace_for(q, B * Hkv, Hq / Hkv, N, D, fmt, W);
  check_rc(fqkv_decode_attn_gqa_strided(q.data_ptr(), K.data_ptr(), V.data_ptr(), quant ? Ks->data_ptr() : nullptr,
                                        quant ? Vs->data_ptr() : nullptr, o.data_ptr(), B, Hq, Hkv, N, D, fmt,
                                        K.stride(0) * elem, K.stride(1) * elem, K.stride(2) * elem,
                                        quant ? Ks->stride(0) : 0, quant ? Ks->stride(1) : 0,
                                        quant ? Ks->stride(2) : 1, W, ws.defined() ? ws.data_ptr() : nullptr,
                                        ws.defined() ? ws.numel() : 0, cur_stream(q)),
           "launch");
  return o;
}

// decode_attn_gqa_paged(q[B,Hq,D], K_pages[P,page_size,Hkv,D or D/2], V_pages, page_table[B,max_pages] int32,
//                       seq_lens[B] int32, max_seq_len, W, Ks_pages=None[P,page_size,Hkv], Vs_pages=None)
// -> o[B,Hq,D]. The page tensors may be any strided view whose last dim is contiguous, so HND
// storage [P,Hkv,page_size,D] is passed as its permute(0,2,1,3).
torch::Tensor decode_attn_gqa_paged(torch::Tensor q, torch::Tensor Kp, torch::Tensor Vp, torch::Tensor page_table,
                                    torch::Tensor seq_lens, int64_t max_seq_len, int64_t W,
                                    c10::optional<torch::Tensor> Ks, c10::optional<torch::Tensor> Vs) {
  check_gpu({&q, &page_table, &seq_lens});
  check_gpu_strided({&Kp, &Vp}, q);
  check_half(q, "q");
  TORCH_CHECK(q.dim() == 3 && Kp.dim() == 4 && Vp.sizes() == Kp.sizes() && Vp.strides() == Kp.strides() &&
                  Vp.scalar_type() == Kp.scalar_type(),
              "shape: expected q [B,Hq,D], K_pages and V_pages [P,page_size,Hkv,D] with equal strides; got q ",
              q.sizes(), ", K_pages ", Kp.sizes());
  TORCH_CHECK(Kp.stride(3) == 1, "contig: the head_dim axis of the pages must be contiguous");
  TORCH_CHECK(page_table.scalar_type() == torch::kInt && seq_lens.scalar_type() == torch::kInt,
              "shape: page_table and seq_lens must be int32");
  TORCH_CHECK(page_table.dim() == 2 && page_table.is_contiguous() && page_table.size(0) == q.size(0) &&
                  seq_lens.dim() == 1 && seq_lens.is_contiguous() && seq_lens.size(0) == q.size(0),
              "shape: expected page_table [B,max_pages] and seq_lens [B], contiguous");
  int64_t D = 0, elem = 0;
  const int fmt = kv_format_of(Kp, &D, &elem);
  check_D(D);
  TORCH_CHECK(q.size(2) == D, "shape: q head_dim ", q.size(2), " does not match KV head_dim ", D);
  const int64_t B = q.size(0), Hq = q.size(1), P = Kp.size(0), page = Kp.size(1), Hkv = Kp.size(2);
  check_W(W);
  TORCH_CHECK(Hkv >= 1 && Hq % Hkv == 0, "heads: Hq (", Hq, ") must be a multiple of Hkv (", Hkv, ")");
  TORCH_CHECK(max_seq_len >= 1, "N: max_seq_len must be >= 1");
  check_scales(fmt, Ks, Vs, {P, page, Hkv});
  const bool qz = quant_fmt(fmt);
  if (qz) TORCH_CHECK(Ks->device() == q.device(), "cuda: all tensors must be on the same device");
  const c10::DeviceGuard guard(q.device());
  auto o = torch::empty({B, Hq, D}, q.options());
  const int64_t max_pages = page_table.size(1);
  const int64_t N = std::min<int64_t>(max_seq_len, max_pages * page);
  auto ws = workspace_for(q, B * Hkv, Hq / Hkv, N, D, fmt, W);
  check_rc(fqkv_decode_attn_gqa_paged(q.data_ptr(), Kp.data_ptr(), Vp.data_ptr(), qz ? Ks->data_ptr() : nullptr,
                                      qz ? Vs->data_ptr() : nullptr, page_table.data_ptr<int32_t>(),
                                      seq_lens.data_ptr<int32_t>(), o.data_ptr(), B, Hq, Hkv, P, max_pages, page,
                                      max_seq_len, D, fmt, Kp.stride(0) * elem, Kp.stride(2) * elem,
                                      Kp.stride(1) * elem, qz ? Ks->stride(0) : 0, qz ? Ks->stride(2) : 0,
                                      qz ? Ks->stride(1) : 1, W, ws.defined() ? ws.data_ptr() : nullptr,
                                      ws.defined() ? ws.numel() : 0, cur_stream(q)),
           "launch");
  return o;
}

// Dequantise int8 [T,D] / int4 [T,D/2] KV through the kernels' conversions.
torch::Tensor dequant_kv(torch::Tensor Kq, torch::Tensor Ks, int64_t path) {
  check_gpu({&Kq, &Ks});
  check_half(Ks, "Ks");
  const bool i8 = Kq.scalar_type() == torch::kChar;
  TORCH_CHECK(i8 || Kq.scalar_type() == torch::kByte, "int8: Kq must be int8 or packed uint8");
  TORCH_CHECK(Kq.dim() >= 2, "shape: Kq must be [..., D] (int8) or [..., D/2] (int4)");
  const int64_t D = i8 ? Kq.size(-1) : 2 * Kq.size(-1);
  check_D(D);
  const int64_t tokens = Kq.numel() / Kq.size(-1);
  TORCH_CHECK(Ks.numel() == tokens, "shape: Ks must hold one scale per token row");
  auto sizes = Kq.sizes().vec();
  sizes.back() = D;
  const c10::DeviceGuard guard(Kq.device());
  auto out = torch::empty(sizes, Kq.options().dtype(torch::kFloat));
  check_rc(fqkv_dequant_kv(Kq.data_ptr(), Ks.data_ptr(), out.data_ptr<float>(), tokens, D,
                           i8 ? FQKV_KV_I8 : FQKV_KV_I4, (int)path, cur_stream(Kq)),
           "launch");
  return out;
}

int64_t choose_splits(int64_t rows, int64_t G, int64_t N, int64_t D, int64_t fmt, int64_t W) {
  return fqkv_choose_splits(rows, G, N, D, (int)fmt, W);
}

int64_t cu_count() {
  int c = 0;
  check_rc(fqkv_device_cu_count(&c), "device");
  return c;
}

}  // namespace

// Per-token KV quantizers on the GPU (fqkv_quantize_kv): the kernel-backed
// producers of the int8 / int4 formats, bit-identical to the reference's
// PyTorch expressions (tests/test_kernels.py:32-34, nb:292-299).
static std::vector<torch::Tensor> quantize_per_token(torch::Tensor X, int fmt) {
  check_gpu({&X});
  TORCH_CHECK(src_of(X) >= 0,
              "fp16: X must be float16, float32 or bfloat16");
  TORCH_CHECK(X.is_contiguous(), "contig: X must be contiguous");
  TORCH_CHECK(X.dim() >= 1, "shape: X must be [..., D]");
  const int64_t D = X.size(-1);
  check_D(D);
  const int64_t tokens = X.numel() / D;
  TORCH_CHECK(tokens >= 1, "shape: X must hold at least one token row");
  const c10::DeviceGuard guard(X.device());
  auto qsizes = X.sizes().vec();
  if (fmt == FQKV_KV_I4) qsizes.back() = D / 2;
  auto Q = torch::empty(qsizes, X.options().dtype(fmt == FQKV_KV_I8   ? torch::kChar
                                                  : fmt == FQKV_KV_FP8 ? torch::kFloat8_e4m3fn
                                                                       : torch::kByte));
  auto ssizes = X.sizes().vec();
  ssizes.pop_back();
  auto S = torch::empty(ssizes, X.options().dtype(torch::kHalf));
  check_rc(fqkv_quantize_kv(X.data_ptr(), src_of(X),
                            Q.data_ptr(), S.data_ptr(), tokens, D, fmt, cur_stream(X)),
           "launch");
  return {Q, S};
}

static std::vector<torch::Tensor> quantize_int8_per_token(torch::Tensor X) {
  return quantize_per_token(X, FQKV_KV_I8);
}
static std::vector<torch::Tensor> quantize_int4_per_token(torch::Tensor X) {
  return quantize_per_token(X, FQKV_KV_I4);
}
static std::vector<torch::Tensor> quantize_fp8_per_token(torch::Tensor X) {
  return quantize_per_token(X, FQKV_KV_FP8);
}

// quantize_kv_append_(K_new[B,H,n,D], V_new, K_cache[B,H,cap,D or D/2], V_cache, Ks_cache[B,H,cap],
// Vs_cache, pos) -> None: quantizes the new tokens into cache positions pos .. pos+n-1 in place.
static void quantize_kv_append(torch::Tensor Kn, torch::Tensor Vn, torch::Tensor Kc, torch::Tensor Vc,
                               torch::Tensor Ksc, torch::Tensor Vsc, int64_t pos) {
  check_gpu({&Kn, &Vn, &Kc, &Vc, &Ksc, &Vsc});
  TORCH_CHECK(src_of(Kn) >= 0,
              "fp16: K_new must be float16, float32 or bfloat16");
  TORCH_CHECK(Vn.scalar_type() == Kn.scalar_type() && Vn.sizes() == Kn.sizes() && Kn.dim() == 4,
              "shape: K_new and V_new must be [B,H,n,D] of one dtype; got ", Kn.sizes(), " and ", Vn.sizes());
  const int fmt = code_format(Kc);
  TORCH_CHECK(fmt >= 0, "int8: caches must be int8, packed uint8 (int4) or float8_e4m3fn");
  const int64_t B = Kn.size(0), H = Kn.size(1), n = Kn.size(2), D = Kn.size(3);
  check_D(D);
  TORCH_CHECK(Kc.dim() == 4 && Kc.size(0) == B && Kc.size(1) == H && Kc.size(3) == (fmt == FQKV_KV_I4 ? D / 2 : D) &&
                  Vc.sizes() == Kc.sizes() && Vc.scalar_type() == Kc.scalar_type(),
              "shape: caches must be [B,H,capacity,", fmt == FQKV_KV_I4 ? "D/2" : "D", "] matching K_new ", Kn.sizes(),
              "; got ", Kc.sizes(), " and ", Vc.sizes());
  const int64_t cap = Kc.size(2);
  check_half(Ksc, "Ks_cache");
  check_half(Vsc, "Vs_cache");
  TORCH_CHECK(Ksc.sizes() == at::IntArrayRef({B, H, cap}) && Vsc.sizes() == Ksc.sizes(),
              "shape: scale caches must be [B,H,capacity] = [", B, ",", H, ",", cap, "]; got ", Ksc.sizes(), " and ",
              Vsc.sizes());
  const c10::DeviceGuard guard(Kn.device());
  check_rc(fqkv_quantize_kv_append(Kn.data_ptr(), Vn.data_ptr(),
                                   src_of(Kn), Kc.data_ptr(),
                                   Vc.data_ptr(), Ksc.data_ptr(), Vsc.data_ptr(), B * H, n, cap, pos, D, fmt,
                                   cur_stream(Kn)),
           "launch");
}

// quantize_kv_append_at_(K_new[B,H,n,D], V_new, K_cache[B,H,cap,D or D/2], V_cache, Ks_cache[B,H,cap],
// Vs_cache, pos[B] int32) -> None: as quantize_kv_append_, sequence b's new tokens at positions
// pos[b] .. pos[b]+n-1, read on the device (graph-capturable); out-of-range rows are not written.
static void quantize_kv_append_at(torch::Tensor Kn, torch::Tensor Vn, torch::Tensor Kc, torch::Tensor Vc,
                                  torch::Tensor Ksc, torch::Tensor Vsc, torch::Tensor pos) {
  check_gpu({&Kn, &Vn, &Kc, &Vc, &Ksc, &Vsc, &pos});
  TORCH_CHECK(src_of(Kn) >= 0,
              "fp16: K_new must be float16, float32 or bfloat16");
  TORCH_CHECK(Vn.scalar_type() == Kn.scalar_type() && Vn.sizes() == Kn.sizes() && Kn.dim() == 4,
              "shape: K_new and V_new must be [B,H,n,D] of one dtype; got ", Kn.sizes(), " and ", Vn.sizes());
  const int fmt = code_format(Kc);
  TORCH_CHECK(fmt >= 0, "int8: caches must be int8, packed uint8 (int4) or float8_e4m3fn");
  const int64_t B = Kn.size(0), H = Kn.size(1), n = Kn.size(2), D = Kn.size(3);
  check_D(D);
  TORCH_CHECK(Kc.dim() == 4 && Kc.size(0) == B && Kc.size(1) == H && Kc.size(3) == (fmt == FQKV_KV_I4 ? D / 2 : D) &&
                  Vc.sizes() == Kc.sizes() && Vc.scalar_type() == Kc.scalar_type(),
              "shape: caches must be [B,H,capacity,", fmt == FQKV_KV_I4 ? "D/2" : "D", "] matching K_new ", Kn.sizes(),
              "; got ", Kc.sizes(), " and ", Vc.sizes());
  const int64_t cap = Kc.size(2);
  check_half(Ksc, "Ks_cache");
  check_half(Vsc, "Vs_cache");
  TORCH_CHECK(Ksc.sizes() == at::IntArrayRef({B, H, cap}) && Vsc.sizes() == Ksc.sizes(),
              "shape: scale caches must be [B,H,capacity] = [", B, ",", H, ",", cap, "]; got ", Ksc.sizes(), " and ",
              Vsc.sizes());
  TORCH_CHECK(pos.scalar_type() == torch::kInt && pos.dim() == 1 && pos.size(0) == B && pos.is_contiguous(),
              "shape: pos must be int32 [B] = [", B, "], contiguous");
  const c10::DeviceGuard guard(Kn.device());
  check_rc(fqkv_quantize_kv_append_at(Kn.data_ptr(), Vn.data_ptr(),
                                      src_of(Kn), Kc.data_ptr(),
                                      Vc.data_ptr(), Ksc.data_ptr(), Vsc.data_ptr(), B * H, n, cap,
                                      pos.data_ptr<int32_t>(), H, D, fmt, cur_stream(Kn)),
           "launch");
}

// quantize_kv_to_pages_(K_new[T,Hkv,D], V_new, slot_mapping[T] int32, K_pages[P,page,Hkv,D or D/2], V_pages,
// Ks_pages[P,page,Hkv], Vs_pages) -> None: token t's K and V rows, quantized as quantize_int8/int4_per_token,
// into slot slot_mapping[t] = page * page_size + offset of the pages decode_attn_gqa_paged reads (any strided
// views with a contiguous last dim, so HND storage passes as .permute(0,2,1,3)); slots outside the pages
// (e.g. -1) are skipped.
static void quantize_kv_to_pages(torch::Tensor Kn, torch::Tensor Vn, torch::Tensor slots, torch::Tensor Kp,
                                 torch::Tensor Vp, torch::Tensor Ksp, torch::Tensor Vsp) {
  check_gpu({&Kn, &Vn, &slots});
  check_gpu_strided({&Kp, &Vp, &Ksp, &Vsp}, Kn);
  TORCH_CHECK(src_of(Kn) >= 0,
              "fp16: K_new must be float16, float32 or bfloat16");
  TORCH_CHECK(Kn.dim() == 3 && Vn.sizes() == Kn.sizes() && Vn.scalar_type() == Kn.scalar_type(),
              "shape: K_new and V_new must be [T,Hkv,D] of one dtype; got ", Kn.sizes(), " and ", Vn.sizes());
  const int fmt = code_format(Kp);
  TORCH_CHECK(fmt >= 0, "int8: pages must be int8, packed uint8 (int4) or float8_e4m3fn");
  const int64_t T = Kn.size(0), H = Kn.size(1), D = Kn.size(2);
  check_D(D);
  TORCH_CHECK(Kp.dim() == 4 && Kp.size(2) == H && Kp.size(3) == (fmt == FQKV_KV_I4 ? D / 2 : D) &&
                  Vp.sizes() == Kp.sizes() && Vp.strides() == Kp.strides() && Vp.scalar_type() == Kp.scalar_type(),
              "shape: pages must be [P,page_size,", H, ",", fmt == FQKV_KV_I4 ? "D/2" : "D",
              "] with equal strides; got ", Kp.sizes(), " and ", Vp.sizes());
  TORCH_CHECK(Kp.stride(3) == 1, "contig: the last dim of the pages must be contiguous");
  check_half(Ksp, "Ks_pages");
  check_half(Vsp, "Vs_pages");
  TORCH_CHECK(Ksp.sizes() == Kp.sizes().slice(0, 3) && Vsp.sizes() == Ksp.sizes() && Vsp.strides() == Ksp.strides(),
              "shape: scale pages must be [P,page_size,Hkv] = ", Kp.sizes().slice(0, 3), " with equal strides; got ",
              Ksp.sizes(), " and ", Vsp.sizes());
  TORCH_CHECK(slots.scalar_type() == torch::kInt && slots.dim() == 1 && slots.size(0) == T,
              "shape: slot_mapping must be int32 [T] = [", T, "]");
  const c10::DeviceGuard guard(Kn.device());
  check_rc(fqkv_quantize_kv_paged(Kn.data_ptr(), Vn.data_ptr(),
                                  src_of(Kn),
                                  slots.data_ptr<int32_t>(), T, H, D, Kp.data_ptr(), Vp.data_ptr(), Ksp.data_ptr(),
                                  Vsp.data_ptr(), Kp.size(0), Kp.size(1), Kp.stride(0), Kp.stride(1), Kp.stride(2),
                                  Ksp.stride(0), Ksp.stride(1), Ksp.stride(2), fmt, cur_stream(Kn)),
           "launch");
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "MI355X fused single-query decode attention (fp16 / int8-KV / int4-KV / GQA / GQA split-K)";
  m.def("decode_attn_fp16_mw", &decode_attn_fp16_mw, "fp16 fused decode", py::arg("q"), py::arg("K"), py::arg("V"),
        py::arg("W"));
  m.def("decode_attn_int8_mw", &decode_attn_int8_mw, "int8-KV fused decode", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("Ks"), py::arg("Vs"), py::arg("W"));
  m.def("decode_attn_int4", &decode_attn_int4, "int4-KV fused decode", py::arg("q"), py::arg("K"), py::arg("V"),
        py::arg("Ks"), py::arg("Vs"), py::arg("W"));
  m.def("decode_attn_gqa", &decode_attn_gqa, "GQA-aware fp16 decode", py::arg("q"), py::arg("K"), py::arg("V"),
        py::arg("W"));
  m.def("gqa_sk_fast", &gqa_sk_fast, "GQA split-K fp16 decode (partial + combine)", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("m_part"), py::arg("l_part"), py::arg("o_part"), py::arg("o"), py::arg("S"),
        py::arg("W"), py::arg("CW"));
  m.def("_gqa_sk_fast_timed", &gqa_sk_fast_timed, "gqa_sk_fast with events around the partial kernel");
  m.def("_dequant_kv", &dequant_kv, "dequantise int8/int4 KV through the kernels' conversions");
  m.def("_probe_stream_read",
        [](torch::Tensor src, int64_t blocks) {
          check_gpu({&src});
          TORCH_CHECK(src.is_contiguous(), "contig: src must be contiguous");
          const c10::DeviceGuard guard(src.device());
          check_rc(fqkv_probe_stream_read(src.data_ptr(), (size_t)src.nbytes(), nullptr, (int)blocks, cur_stream(src)),
                   "launch");
        },
        "read a tensor once with streaming loads (the bandwidth ceiling of a decode call)");
  m.def("decode_attn_gqa_int8", &decode_attn_gqa_int8, "GQA-aware int8-KV decode", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("Ks"), py::arg("Vs"), py::arg("W"));
  m.def("decode_attn_gqa_int4", &decode_attn_gqa_int4, "GQA-aware int4-KV decode", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("Ks"), py::arg("Vs"), py::arg("W"));
  m.def("gqa_sk_fast_int8", &gqa_sk_fast_int8, "GQA split-K int8-KV decode", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("Ks"), py::arg("Vs"), py::arg("m_part"), py::arg("l_part"), py::arg("o_part"),
        py::arg("o"), py::arg("S"), py::arg("W"), py::arg("CW"));
  m.def("gqa_sk_fast_int4", &gqa_sk_fast_int4, "GQA split-K int4-KV decode", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("Ks"), py::arg("Vs"), py::arg("m_part"), py::arg("l_part"), py::arg("o_part"),
        py::arg("o"), py::arg("S"), py::arg("W"), py::arg("CW"));
  m.def("gqa_sk_fast_bf16", &gqa_sk_fast_bf16, "GQA split-K decode over bf16 K and V", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("m_part"), py::arg("l_part"), py::arg("o_part"), py::arg("o"), py::arg("S"),
        py::arg("W"), py::arg("CW"));
  m.def("decode_attn_gqa_fp8", &decode_attn_gqa_fp8, "GQA-aware fp8 (e4m3) KV decode", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("Ks"), py::arg("Vs"), py::arg("W"));
  m.def("gqa_sk_fast_fp8", &gqa_sk_fast_fp8, "GQA split-K fp8 (e4m3) KV decode", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("Ks"), py::arg("Vs"), py::arg("m_part"), py::arg("l_part"), py::arg("o_part"),
        py::arg("o"), py::arg("S"), py::arg("W"), py::arg("CW"));
  m.def("decode_attn_gqa_nhd", &decode_attn_gqa_nhd, "GQA decode over a token-major [B,N,Hkv,D] KV cache",
        py::arg("q"), py::arg("K"), py::arg("V"), py::arg("W"), py::arg("Ks") = py::none(),
        py::arg("Vs") = py::none());
  m.def("decode_attn_gqa_strided", &decode_attn_gqa_strided,
        "GQA decode over [B,Hkv,N,D] KV views with any strides (contiguous rows)", py::arg("q"), py::arg("K"),
        py::arg("V"), py::arg("W"), py::arg("Ks") = py::none(), py::arg("Vs") = py::none());
  m.def("decode_attn_gqa_paged", &decode_attn_gqa_paged, "GQA decode over a paged KV cache", py::arg("q"),
        py::arg("K_pages"), py::arg("V_pages"), py::arg("page_table"), py::arg("seq_lens"), py::arg("max_seq_len"),
        py::arg("W"), py::arg("Ks_pages") = py::none(), py::arg("Vs_pages") = py::none());
  m.def("quantize_int8_per_token", &quantize_int8_per_token,
        "per-token int8 KV quantizer on the GPU -> (int8 [..., D], fp16 scales [...])", py::arg("X"));
  m.def("quantize_int4_per_token", &quantize_int4_per_token,
        "per-token int4 KV quantizer on the GPU -> (packed uint8 [..., D/2], fp16 scales [...])", py::arg("X"));
  m.def("quantize_fp8_per_token", &quantize_fp8_per_token,
        "per-token fp8 e4m3 KV quantizer on the GPU -> (float8_e4m3fn [..., D], fp16 scales [...])", py::arg("X"));
  m.def("quantize_kv_append_", &quantize_kv_append,
        "quantize new K/V tokens [B,H,n,D] into int8 / int4 caches [B,H,capacity,.] at position pos, in place",
        py::arg("K_new"), py::arg("V_new"), py::arg("K_cache"), py::arg("V_cache"), py::arg("Ks_cache"),
        py::arg("Vs_cache"), py::arg("pos"));
  m.def("quantize_kv_append_at_", &quantize_kv_append_at,
        "quantize_kv_append_ with each sequence's position read on the device from pos [B] int32 (graph-capturable)",
        py::arg("K_new"), py::arg("V_new"), py::arg("K_cache"), py::arg("V_cache"), py::arg("Ks_cache"),
        py::arg("Vs_cache"), py::arg("pos"));
  m.def("quantize_kv_to_pages_", &quantize_kv_to_pages,
        "quantize new K and V tokens into paged int8 / int4 caches at their slots (in place)", py::arg("K_new"),
        py::arg("V_new"), py::arg("slot_mapping"), py::arg("K_pages"), py::arg("V_pages"), py::arg("Ks_pages"),
        py::arg("Vs_pages"));
  m.def("_choose_splits", &choose_splits, "split count the single-block entry points use");
  m.def("_cu_count", &cu_count, "compute units of the current device");
  m.def("_version", []() { return std::string(fqkv_version()); });
  m.def("_set_pv_valu", [](bool enable) { fqkv_set_pv_valu(enable ? 1 : 0); },
        "measurement knob: P.V on the vector ALUs (fp16, D 128, 1 or 4 heads per group, contiguous rows)");
  m.def("_set_two_kernel_merge", [](bool enable) { fqkv_set_two_kernel_merge(enable ? 1 : 0); },
        "force the two-kernel split merge (testing / comparison)");
  m.def("_last_merge_protocol", []() { return fqkv_last_merge_protocol(); },
        "split merge of this thread's last call: 0 none, 1 two-kernel, 2 device scope, 3 XCD-local");
  m.def("_merge_fallback_count", []() { return fqkv_merge_fallback_count(); },
        "calls that took the two-kernel merge because no counter slot was free");
  m.def("_xcd_period", [](int device) { return fqkv_xcd_period(device); },
        "XCD period the probe found (> 0), 0 before the probe, -1 when unusable");
  m.def("_release_capture_slots", []() {
        const int rc = fqkv_release_capture_slots();
        TORCH_CHECK(rc == FQKV_OK, "release_capture_slots: ", fqkv_last_error());
      },
        "free the capture slots of the current device (after destroying every graph that used them)");
}
