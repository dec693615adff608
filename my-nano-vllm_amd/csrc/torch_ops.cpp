// The attention path as C++ operators of torch's dispatcher (host code only,
// no device code): torch.ops.nvamd.store_kvcache, torch.ops.nvamd.decode and
// torch.ops.nvamd.prefill, for the reference's three attention calls, and
// torch.ops.nvamd.fp8_block_linear for its FP8 linear layer
//   store_kvcache          nanovllm/layers/attention.py:33-40
//   fp8_decode_attention   nanovllm/kernels/fp8_attention.py:173-207
//   fp8_prefill_attention  nanovllm/kernels/fp8_attention.py:314-353
//   fp8_block_linear       nanovllm/kernels/fp8_linear.py:93-139
// The argument checks, the output and workspace allocations (torch's caching
// allocator) and the launches through the C ABI
// (include/nvamd_fp8_attention.h, nvamd_fp8_linear.h) run here, so a call from Python costs one
// dispatcher hop instead of Python checks plus ctypes marshalling.  Kernels
// are enqueued on torch's current stream of the tensors' device; nothing
// synchronises, so the operators can be captured in a HIP graph.
//
// Errors: invalid arguments raise ValueError (TORCH_CHECK_VALUE), a failing
// library call RuntimeError with the library's message.  Meta kernels give
// FakeTensor / torch.compile tracing the output shapes.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "nvamd_fp8_attention.h"
#include "nvamd_fp8_linear.h"

namespace {

void check_gpu(const at::Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(t.is_cuda(), name, " must be on a ROCm GPU (got ", t.device(), ")");
}

int32_t qo_dtype(const at::Tensor& q, const char* name) {
  TORCH_CHECK_VALUE(q.scalar_type() == at::kBFloat16 || q.scalar_type() == at::kHalf, name,
                    " must be bfloat16 or float16 (got ", q.scalar_type(), ")");
  return q.scalar_type() == at::kHalf ? NVAMD_DTYPE_F16 : NVAMD_DTYPE_BF16;
}

void check_fp8(const at::Tensor& t, const char* name) {
  check_gpu(t, name);
  TORCH_CHECK_VALUE(t.scalar_type() == at::kFloat8_e4m3fn, name, " must be float8_e4m3fn (got ", t.scalar_type(),
                    ")");
}

at::Tensor int32_contig(const at::Tensor& t, const char* name) {
  check_gpu(t, name);
  return (t.scalar_type() == at::kInt ? t : t.to(at::kInt)).contiguous();
}

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// The kernels take at most 32 query heads per kv head (G; the decode kernels
// hold G query columns of a kv head in two 16-column MFMA blocks).  The
// reference's kernels take any G, so a call with more runs as G / gs calls,
// gs the largest divisor of G up to 32: call s takes query heads
// j G + s gs .. j G + s gs + gs - 1 of every kv head j, as a contiguous copy
// in which kv head j owns query heads j gs .. j gs + gs - 1, and its output
// is copied back into those heads.  Each call streams the K/V again.  Returns
// gs, or 0 when no split is needed (or the shapes are invalid: the checks of
// the unsplit call report them).
constexpr int64_t kMaxHeadsPerKvHead = 32;
int64_t head_slice(int64_t num_heads, int64_t num_kv_heads) {
  if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return 0;
  const int64_t g = num_heads / num_kv_heads;
  if (g <= kMaxHeadsPerKvHead) return 0;
  int64_t gs = kMaxHeadsPerKvHead;
  while (g % gs != 0) --gs;
  return gs;
}

// out[:, heads of slice s] = call(q[:, heads of slice s]) for every slice (see head_slice).
template <typename F>
void run_head_slices(const at::Tensor& q, at::Tensor& out, int64_t num_kv_heads, int64_t gs, F&& call) {
  const int64_t rows = q.size(0), g = q.size(1) / num_kv_heads, d = q.size(2);
  const at::Tensor qv = q.view({rows, num_kv_heads, g / gs, gs, d});
  at::Tensor ov = out.view({rows, num_kv_heads, g / gs, gs, d});
  for (int64_t s = 0; s < g / gs; ++s) {
    const at::Tensor qs = qv.select(2, s).reshape({rows, num_kv_heads * gs, d});
    ov.select(2, s).copy_(call(qs).view({rows, num_kv_heads, gs, d}));
  }
}

void check_status(int32_t st, const char* what) {
  TORCH_CHECK(st == NVAMD_OK, what, " failed (status ", st, "): ", nvamd_last_error());
}

// Scratch straight from torch's caching allocator on the current device (no
// tensor, no dispatcher call); freed when the call returns, which the
// allocator orders after the work already enqueued on the stream.
c10::DataPtr workspace(int64_t nbytes) {
  if (nbytes <= 0) return c10::DataPtr();
  return c10::hip::HIPCachingAllocator::get()->allocate((size_t)nbytes);
}

// attention.py:33-40, with the reference's assertions.
void store_kvcache(const at::Tensor& key, const at::Tensor& value, const at::Tensor& k_cache,
                   const at::Tensor& v_cache, const at::Tensor& slot_mapping) {
  TORCH_CHECK_VALUE(key.dim() == 3, "key must be [N, num_kv_heads, head_dim]");
  const int64_t N = key.size(0), heads = key.size(1), head_dim = key.size(2), D = heads * head_dim;
  TORCH_CHECK_VALUE(key.stride(-1) == 1 && value.stride(-1) == 1, "key/value rows must be contiguous");
  TORCH_CHECK_VALUE(key.stride(1) == head_dim && value.stride(1) == head_dim, "key/value heads must be packed");
  TORCH_CHECK_VALUE(k_cache.dim() >= 2 && k_cache.stride(1) == D && v_cache.dim() >= 2 && v_cache.stride(1) == D,
                    "cache rows must hold num_kv_heads * head_dim elements");
  TORCH_CHECK_VALUE(slot_mapping.numel() == N, "slot_mapping must have one entry per token");
  check_gpu(key, "key");
  check_gpu(value, "value");
  check_fp8(k_cache, "k_cache");
  check_fp8(v_cache, "v_cache");
  TORCH_CHECK_VALUE(value.sizes() == key.sizes(), "key and value shapes differ");
  const int32_t dt = qo_dtype(key, "key");
  TORCH_CHECK_VALUE(value.scalar_type() == key.scalar_type(), "key and value must have the same dtype");
  TORCH_CHECK_VALUE(k_cache.is_contiguous() && v_cache.is_contiguous(), "k_cache/v_cache must be contiguous");
  const at::Tensor slots = int32_contig(slot_mapping, "slot_mapping");
  const at::OptionalDeviceGuard guard(key.device());
  check_status(nvamd_store_kvcache(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
                                   k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr<int32_t>(), N,
                                   (int32_t)heads, (int32_t)head_dim, k_cache.numel() / D, dt, stream_of(key)),
               "store_kvcache");
}

// fp8_attention.py:173-207.
at::Tensor decode(const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& v_in,
                  const at::Tensor& block_tables_in, const at::Tensor& context_lens_in, double softmax_scale) {
  check_gpu(q_in, "q");
  const int32_t dt = qo_dtype(q_in, "q");
  check_fp8(k_in, "k_cache");
  check_fp8(v_in, "v_cache");
  TORCH_CHECK_VALUE(q_in.dim() == 3, "q must be [batch, num_heads, head_dim]");
  TORCH_CHECK_VALUE(k_in.dim() == 4 && v_in.sizes() == k_in.sizes(),
                    "k_cache/v_cache must be [num_blocks, block_size, num_kv_heads, head_dim]");
  const int64_t num_heads = q_in.size(1);
  const int64_t num_blocks = k_in.size(0), block_size = k_in.size(1), num_kv_heads = k_in.size(2);
  const int64_t head_dim = k_in.size(3);
  TORCH_CHECK_VALUE(q_in.size(2) == head_dim, "q head_dim does not match the cache");
  const at::Tensor bt = int32_contig(block_tables_in, "block_tables");
  const at::Tensor ctx = int32_contig(context_lens_in, "context_lens");
  TORCH_CHECK_VALUE(bt.dim() == 2, "block_tables must be [batch, max_num_blocks]");
  const int64_t batch = bt.size(0), max_num_blocks = bt.size(1);
  TORCH_CHECK_VALUE(q_in.size(0) >= batch && ctx.numel() >= batch,
                    "q and context_lens need at least block_tables.shape[0] rows");
  const at::Tensor q = q_in.contiguous(), k = k_in.contiguous(), v = v_in.contiguous();
  at::Tensor out = at::empty(q.sizes(), q.options());
  if (batch == 0) return out;
  if (const int64_t gs = head_slice(num_heads, num_kv_heads)) {
    run_head_slices(q, out, num_kv_heads, gs,
                    [&](const at::Tensor& qs) { return decode(qs, k, v, bt, ctx, softmax_scale); });
    return out;
  }
  const at::OptionalDeviceGuard guard(q.device());
  const int64_t ws_n = nvamd_decode_workspace_bytes((int32_t)batch, (int32_t)num_heads, (int32_t)num_kv_heads,
                                                    (int32_t)max_num_blocks, (int32_t)block_size, 0);
  const c10::DataPtr ws = workspace(ws_n);
  check_status(nvamd_fp8_decode_attention(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                          bt.data_ptr<int32_t>(), ctx.data_ptr<int32_t>(), (int32_t)batch,
                                          (int32_t)num_heads, (int32_t)num_kv_heads, (int32_t)head_dim, num_blocks,
                                          (int32_t)block_size, (int32_t)max_num_blocks, (float)softmax_scale, 0,
                                          ws.get(), ws.get() != nullptr ? ws_n : 0, dt, stream_of(q)),
               "fp8_decode_attention");
  return out;
}

// fp8_attention.py:314-353.
at::Tensor prefill(const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& v_in,
                   const c10::optional<at::Tensor>& block_tables_in, const at::Tensor& cu_q_in,
                   const at::Tensor& cu_k_in, int64_t max_seqlen_q, int64_t max_seqlen_k, double softmax_scale) {
  check_gpu(q_in, "q");
  const int32_t dt = qo_dtype(q_in, "q");
  check_fp8(k_in, "k");
  check_fp8(v_in, "v");
  TORCH_CHECK_VALUE(q_in.dim() == 3, "q must be [num_tokens, num_heads, head_dim]");
  const int64_t num_tokens = q_in.size(0), num_heads = q_in.size(1), head_dim = q_in.size(2);
  const at::Tensor cu_q = int32_contig(cu_q_in, "cu_seqlens_q");
  const at::Tensor cu_k = int32_contig(cu_k_in, "cu_seqlens_k");
  const int64_t num_seqs = cu_q.size(0) - 1;
  TORCH_CHECK_VALUE(cu_k.size(0) == num_seqs + 1, "cu_seqlens_k must have num_seqs + 1 entries");
  const bool paged = block_tables_in.has_value() && block_tables_in->defined();
  int64_t num_kv_heads, num_kv_rows, block_size = 0, max_num_blocks = 0, kv_cap;
  at::Tensor bt;
  if (!paged) {
    TORCH_CHECK_VALUE(k_in.dim() == 3 && v_in.sizes() == k_in.sizes(),
                      "contiguous k/v must be [num_kv_tokens, num_kv_heads, head_dim]");
    num_kv_heads = k_in.size(1);
    num_kv_rows = k_in.size(0);
    kv_cap = num_kv_rows;
  } else {
    TORCH_CHECK_VALUE(k_in.dim() == 4 && v_in.sizes() == k_in.sizes(),
                      "paged k/v must be [num_blocks, block_size, num_kv_heads, head_dim]");
    bt = int32_contig(*block_tables_in, "block_tables");
    TORCH_CHECK_VALUE(bt.dim() == 2 && bt.size(0) >= num_seqs, "block_tables needs a row per sequence");
    block_size = k_in.size(1);
    num_kv_heads = k_in.size(2);
    num_kv_rows = k_in.size(0) * block_size;
    max_num_blocks = bt.size(1);
    kv_cap = max_num_blocks * block_size;
  }
  TORCH_CHECK_VALUE(k_in.size(-1) == head_dim, "k head_dim does not match q");
  const at::Tensor q = q_in.contiguous(), k = k_in.contiguous(), v = v_in.contiguous();
  at::Tensor out = at::empty(q.sizes(), q.options());
  if (num_tokens == 0 || num_seqs <= 0) return out;
  if (const int64_t gs = head_slice(num_heads, num_kv_heads)) {
    run_head_slices(q, out, num_kv_heads, gs, [&](const at::Tensor& qs) {
      return prefill(qs, k, v, block_tables_in, cu_q, cu_k, max_seqlen_q, max_seqlen_k, softmax_scale);
    });
    return out;
  }
  const at::OptionalDeviceGuard guard(q.device());
  const int64_t ws_n = nvamd_prefill_workspace_bytes(num_tokens, (int32_t)num_seqs, (int32_t)num_heads,
                                                     (int32_t)num_kv_heads, kv_cap, (int32_t)max_seqlen_q,
                                                     (int32_t)block_size, 0);
  const c10::DataPtr ws = workspace(ws_n);
  check_status(nvamd_fp8_prefill_attention(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                           paged ? bt.data_ptr<int32_t>() : nullptr, cu_q.data_ptr<int32_t>(),
                                           cu_k.data_ptr<int32_t>(), num_tokens, (int32_t)num_seqs,
                                           (int32_t)num_heads, (int32_t)num_kv_heads, (int32_t)head_dim,
                                           num_kv_rows, (int32_t)block_size, (int32_t)max_num_blocks,
                                           (int32_t)max_seqlen_q, (int32_t)max_seqlen_k, (float)softmax_scale, 0,
                                           ws.get(), ws.get() != nullptr ? ws_n : 0, dt, stream_of(q)),
               "fp8_prefill_attention");
  return out;
}

// fp8_linear.py:93-139: the per-token, per-128-column activation
// quantisation, then the 128 x 128 block-scaled GEMM; y = x @ weight.T in x's
// dtype.
at::Tensor fp8_block_linear(const at::Tensor& x_in, const at::Tensor& w_in, const at::Tensor& ws_in) {
  check_gpu(x_in, "x");
  const int32_t dt = qo_dtype(x_in, "x");
  check_fp8(w_in, "weight");
  check_gpu(ws_in, "weight_scale");
  TORCH_CHECK_VALUE(x_in.dim() == 2 && w_in.dim() == 2 && ws_in.dim() == 2,
                    "x [M, K], weight [N, K] and weight_scale [N/128, K/128] are matrices");
  const int64_t M = x_in.size(0), K = x_in.size(1), N = w_in.size(0);
  TORCH_CHECK_VALUE(w_in.size(1) == K, "weight must be [N, K]");
  TORCH_CHECK_VALUE(N == ws_in.size(0) * 128 && K == ws_in.size(1) * 128,
                    "weight_scale must be [N/128, K/128] (128 x 128 weight blocks)");
  const at::Tensor x = (x_in.stride(1) != 1 || x_in.stride(0) % 8 != 0 ||
                        reinterpret_cast<uintptr_t>(x_in.data_ptr()) % 16 != 0)
                           ? x_in.contiguous()
                           : x_in;
  const at::Tensor w = (w_in.stride(1) != 1 || w_in.stride(0) % 16 != 0 ||
                        reinterpret_cast<uintptr_t>(w_in.data_ptr()) % 16 != 0)
                           ? w_in.contiguous()
                           : w_in;
  const at::Tensor wsc = (ws_in.scalar_type() == at::kBFloat16 ? ws_in : ws_in.to(at::kBFloat16)).contiguous();
  const at::OptionalDeviceGuard guard(x.device());
  const hipStream_t stream = stream_of(x);
  // the quantised activations [M, K] and their bf16 scales [M, K/128], one allocation
  const int64_t xq_bytes = (M * K + 255) / 256 * 256;
  const c10::DataPtr act = workspace(xq_bytes + M * (K / 128) * 2);
  void* xq = act.get();
  void* x_scale = static_cast<char*>(act.get()) + xq_bytes;
  check_status(nvamd_fp8_act_quant(x.data_ptr(), x.stride(0), dt, xq, x_scale, M, K, stream), "fp8_act_quant");
  at::Tensor out = at::empty({M, N}, x.options());
  const int64_t ws_n = nvamd_fp8_block_gemm_workspace_bytes(M, N, K);
  const c10::DataPtr ws = workspace(ws_n);
  check_status(nvamd_fp8_block_gemm(xq, x_scale, w.data_ptr(), w.stride(0), wsc.data_ptr(), out.data_ptr(),
                                    out.stride(0), dt, M, N, K, ws.get(), ws.get() != nullptr ? ws_n : 0, stream),
               "fp8_block_gemm");
  return out;
}

void store_kvcache_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                        const at::Tensor&) {}

at::Tensor decode_meta(const at::Tensor& q, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                       const at::Tensor&, double) {
  return at::empty_like(q);
}

at::Tensor fp8_block_linear_meta(const at::Tensor& x, const at::Tensor& w, const at::Tensor&) {
  return at::empty({x.size(0), w.size(0)}, x.options());
}

at::Tensor prefill_meta(const at::Tensor& q, const at::Tensor&, const at::Tensor&, const c10::optional<at::Tensor>&,
                        const at::Tensor&, const at::Tensor&, int64_t, int64_t, double) {
  return at::empty_like(q);
}

}  // namespace

TORCH_LIBRARY(nvamd, m) {
  m.def("store_kvcache(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor slot_mapping) -> ()");
  m.def("decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, Tensor context_lens, float scale) "
        "-> Tensor");
  m.def("prefill(Tensor q, Tensor k, Tensor v, Tensor? block_tables, Tensor cu_q, Tensor cu_k, SymInt max_q, "
        "SymInt max_k, float scale) -> Tensor");
  m.def("fp8_block_linear(Tensor x, Tensor weight, Tensor weight_scale) -> Tensor");
}

TORCH_LIBRARY_IMPL(nvamd, CUDA, m) {
  m.impl("store_kvcache", &store_kvcache);
  m.impl("decode", &decode);
  m.impl("prefill", &prefill);
  m.impl("fp8_block_linear", &fp8_block_linear);
}

TORCH_LIBRARY_IMPL(nvamd, Meta, m) {
  m.impl("store_kvcache", &store_kvcache_meta);
  m.impl("decode", &decode_meta);
  m.impl("prefill", &prefill_meta);
  m.impl("fp8_block_linear", &fp8_block_linear_meta);
}
