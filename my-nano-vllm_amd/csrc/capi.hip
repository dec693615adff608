// C ABI entry points (declared in include/nvamd_fp8_attention.h,
// include/nvamd_fp8_linear.h and include/nvamd_lm_head.h): argument
// validation, static partition sizing and kernel launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "kernels.h"
#include "nvamd_fp8_attention.h"
#include "nvamd_fp8_linear.h"
#include "nvamd_lm_head.h"

// Scratch of nvamd_fp8_decode_attention_noalloc: device memory the library
// holds for the whole process on every GPU it runs on (each GPU has its own
// copy of the array at its own address).  Host code never uses the array's
// name as an address (it is a host-side stand-in): the device address comes
// from hipGetSymbolAddress, once per device (noalloc_scratch below).
static __device__ __align__(256) uint8_t scratch[NVAMD_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int32_t ok() {
  g_last_error.clear();
  return NVAMD_OK;
}

int32_t launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(NVAMD_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

// Device address of `scratch` on the current device, looked up on the first
// call on that device (with it current) and kept per device.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

int32_t noalloc_scratch(const char* fn, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NVAMD_ERR_LAUNCH, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: device ordinal %d beyond %d", fn, dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(NVAMD_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev].store(p, std::memory_order_release);  // the same address if two threads race here
  }
  *out = p;
  return NVAMD_OK;
}

// CUs of the current device, looked up once per device (every host call
// sizes its grid and workspace from it).
std::atomic<int> g_cu_count[kMaxDevices];

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  const bool cached = dev >= 0 && dev < kMaxDevices;
  if (cached) {
    const int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  if (cached) g_cu_count[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

constexpr int kHeadDim = 128;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
constexpr int kMqMaxCols = 32;        // query rows per kv head packed by the split-KV kernel
constexpr int kPartAlign = 256;       // partition lengths are multiples of 256 tokens
constexpr int64_t kPartialFloats = kHeadDim + 2;  // acc[128] + (m, l) per partition

// A paged partition spans at most this many KV blocks: the decode kernel
// holds the partition's block-table entries in one wave-wide register
// (64 lanes; one spare for a partition that starts inside a block).
constexpr int64_t kMaxPartBlocks = 63;

int64_t max_part_tokens(int32_t block_size) {
  if (block_size <= 0) return INT64_MAX;  // contiguous layout: no table
  return kMaxPartBlocks * block_size / kPartAlign * kPartAlign;
}

// kv heads per decode workgroup (the kernel reads HG*128-byte row slices).
int64_t kv_head_groups(int32_t num_kv_heads) {
  return (num_kv_heads % 2 == 0) ? num_kv_heads / 2 : num_kv_heads;
}

// Split-KV partition length from static shapes only (graph-safe): aim for
// about 4 workgroups per CU when every sequence is at its capacity, within
// the block-table limit of a partition.
int64_t choose_part_tokens(int64_t items, int64_t kv_cap, int64_t requested, int32_t block_size) {
  if (requested > 0) return requested;
  const int64_t cap = max_part_tokens(block_size);
  items = std::max<int64_t>(items, 1);
  const int64_t target = (int64_t)device_cu_count() * 4;
  const int64_t parts = std::max<int64_t>((target + items - 1) / items, 1);
  int64_t part = (std::max<int64_t>(kv_cap, 1) + parts - 1) / parts;
  part = (part + kPartAlign - 1) / kPartAlign * kPartAlign;
  return std::min(std::max<int64_t>(part, kPartAlign), cap);
}

int64_t partial_bytes(int64_t rows, int64_t heads, int64_t max_parts) {
  if (max_parts <= 1) return 0;
  return rows * heads * max_parts * kPartialFloats * (int64_t)sizeof(float);
}

// Balanced (stream-K) decode: used when the caller leaves the partition to
// the library, the kv heads split into groups of 4 and the batch fits the
// kernel's in-LDS stage prefix.
bool use_stream_k(int32_t batch, int32_t num_kv_heads, int32_t part_tokens) {
  return part_tokens == 0 && num_kv_heads % 4 == 0 && batch <= nvamd::kSkMaxSeqs;
}

// Query columns per kv head of the short-query rows of a varlen call.
int short_cols(int G, int32_t max_seqlen_q) { return G * std::min(32 / G, std::max(max_seqlen_q, 1)); }

// kv heads per balanced-decode workgroup: whole 1 KiB cache rows when the
// kv heads come in 8s (each workgroup then reads whole DRAM pages), else 4.
// The short-query rows of a varlen call take 4: their workgroups read
// their queries from global memory, which drains the ring at each pair
// switch, and with 4 heads two half-size workgroups share a CU, so one keeps
// streaming while the other drains.
int stream_k_heads(int32_t num_kv_heads, bool varlen) { return num_kv_heads % 8 == 0 && !varlen ? 8 : 4; }

int stream_k_wgs(int ncb, int hg, int G, bool varlen) {
  return device_cu_count() * nvamd::decode_sk_wgs_per_cu(ncb, hg, G, varlen);
}

// Workspace of the balanced kernel: the stage prefix, then the partial slots
// (cols query columns per kv head: G for decode, G * mq_max_q for the
// short-query rows of a varlen call).
int64_t stream_k_prefix_bytes(int32_t batch) { return (((int64_t)batch + 1) * 4 + 255) / 256 * 256; }
int64_t stream_k_bytes(int32_t batch, int32_t num_kv_heads, int32_t G, int cols, bool varlen) {
  const int ncb = (cols + 15) / 16, hg = stream_k_heads(num_kv_heads, varlen);
  return stream_k_prefix_bytes(batch) +
         (int64_t)stream_k_wgs(ncb, hg, G, varlen) * 2 * hg * cols * nvamd::kSkSlotFloats * (int64_t)sizeof(float);
}

void set_partials(nvamd::MqParams& p, void* workspace) {
  const int64_t n = p.q_rows * p.Hq * p.max_parts;
  p.part_acc = static_cast<float*>(workspace);
  p.part_ml = p.part_acc ? p.part_acc + n * kHeadDim : nullptr;
}

int32_t check_qo_dtype(const char* fn, int32_t qo_dtype) {
  if (qo_dtype != NVAMD_DTYPE_BF16 && qo_dtype != NVAMD_DTYPE_F16)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: qo_dtype must be bf16 or fp16 (got %d)", fn, qo_dtype);
  return NVAMD_OK;
}

int32_t check_heads(const char* fn, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim) {
  if (head_dim != kHeadDim)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: head_dim must be %d (got %d)", fn, kHeadDim, head_dim);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: num_heads (%d) must be a positive multiple of num_kv_heads (%d)",
                fn, num_heads, num_kv_heads);
  return NVAMD_OK;
}

// Largest power of two <= 4 dividing g: query heads per prefill workgroup.
int heads_per_workgroup(int g) {
  if (g % 4 == 0) return 4;
  if (g % 2 == 0) return 2;
  return 1;
}

int64_t align_up(int64_t n) { return (n + 255) / 256 * 256; }

// Prefill kernel geometry for G query heads per kv head.
int prefill_bm(int g) { return 32 * nvamd::kPrefillWaves / heads_per_workgroup(g); }

constexpr int64_t kPrefillItemBytes = 48;  // sizeof(nvamd::PrefillItem)

// Workspace of the prefill kernel after the short-query partials: the work
// list, the arrival counters of split items and the partial slots of their
// pieces (all 0 when every sequence takes the short-query path).
struct PrefillLayout {
  int64_t records = 0, slots_per_group = 0, list_bytes = 0, counter_bytes = 0, part_bytes = 0;
  int64_t bytes() const { return list_bytes + counter_bytes + part_bytes; }
};

PrefillLayout prefill_layout(int32_t num_seqs, int32_t num_kv_heads, int g, int32_t max_seqlen_q) {
  PrefillLayout L;
  if (max_seqlen_q <= kMqMaxCols / g) return L;
  const int64_t n_items = (int64_t)num_seqs * ceil_div(max_seqlen_q, prefill_bm(g));
  const int64_t n_groups = (int64_t)num_kv_heads * (g / heads_per_workgroup(g));
  L.slots_per_group = std::max<int64_t>(1, device_cu_count() / n_groups);
  L.records = std::max(n_items, 2 * L.slots_per_group);
  L.list_bytes = align_up(L.records * kPrefillItemBytes);
  L.counter_bytes = align_up((L.slots_per_group * n_groups + 3) * (int64_t)sizeof(int));
  L.part_bytes = 2 * L.slots_per_group * n_groups * nvamd::kPrefillPartDwords * 64 * nvamd::kPrefillWaves *
                 (int64_t)sizeof(uint32_t);
  return L;
}

}  // namespace

extern "C" {

int32_t nvamd_abi_version(void) { return NVAMD_ABI_VERSION; }

const char* nvamd_last_error(void) { return g_last_error.c_str(); }

int32_t nvamd_store_kvcache(const void* key, int64_t key_stride0, const void* value,
                            int64_t value_stride0, void* k_cache, void* v_cache,
                            const int32_t* slot_mapping, int64_t num_tokens, int32_t num_kv_heads,
                            int32_t head_dim, int64_t num_slots, int32_t kv_dtype, void* stream) {
  if (kv_dtype != NVAMD_DTYPE_BF16 && kv_dtype != NVAMD_DTYPE_F16)
    return fail(NVAMD_ERR_UNSUPPORTED, "store_kvcache: kv_dtype must be bf16 or fp16 (got %d)", kv_dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_slots < 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "store_kvcache: bad sizes (N=%lld Hkv=%d D=%d slots=%lld)",
                (long long)num_tokens, num_kv_heads, head_dim, (long long)num_slots);
  if (num_tokens == 0) return ok();
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "store_kvcache: null pointer");
  const int row = num_kv_heads * head_dim;
  const bool vec = (row % 16 == 0) && (key_stride0 % 8 == 0) && (value_stride0 % 8 == 0) &&
                   ((uintptr_t)key % 16 == 0) && ((uintptr_t)value % 16 == 0) &&
                   ((uintptr_t)k_cache % 16 == 0) && ((uintptr_t)v_cache % 16 == 0);
  return launch_status(nvamd::launch_kv_store(key, key_stride0, value, value_stride0, k_cache, v_cache,
                                              slot_mapping, num_tokens, row, num_slots, vec,
                                              kv_dtype == NVAMD_DTYPE_F16, (hipStream_t)stream),
                       "store_kvcache");
}

int32_t nvamd_qk_norm_rope_store(const void* qkv, int64_t qkv_stride0, const int64_t* positions,
                                 const void* q_norm_weight, const void* k_norm_weight, float eps,
                                 const float* cos_sin_cache, int64_t max_position, void* q_out, void* k_out,
                                 void* k_cache, void* v_cache, const int32_t* slot_mapping, int64_t num_tokens,
                                 int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                                 void* stream) {
  static const char* fn = "qk_norm_rope_store";
  if (head_dim != kHeadDim)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: head_dim must be %d (got %d)", fn, kHeadDim, head_dim);
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_slots < 0 || max_position <= 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: bad sizes (N=%lld Hq=%d Hkv=%d slots=%lld max_position=%lld)", fn,
                (long long)num_tokens, num_heads, num_kv_heads, (long long)num_slots, (long long)max_position);
  if (!(eps >= 0.f) || !std::isfinite(eps))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: eps must be finite and non-negative", fn);
  if (num_heads + 2 * num_kv_heads > 128)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: at most 128 head rows per token (num_heads + 2 * num_kv_heads = %d)", fn,
                num_heads + 2 * num_kv_heads);
  if (qkv_stride0 < (int64_t)(num_heads + 2 * num_kv_heads) * head_dim)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: qkv row stride %lld is shorter than a row", fn, (long long)qkv_stride0);
  if (num_tokens == 0) return ok();
  if (!qkv || !positions || !q_norm_weight || !k_norm_weight || !cos_sin_cache || !q_out ||
      (num_slots > 0 && (!k_cache || !v_cache || !slot_mapping)))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (qkv_stride0 % 8 != 0 || (uintptr_t)qkv % 16 != 0 || (uintptr_t)q_out % 16 != 0 ||
      (k_out && (uintptr_t)k_out % 16 != 0) || (uintptr_t)q_norm_weight % 16 != 0 ||
      (uintptr_t)k_norm_weight % 16 != 0 || (uintptr_t)cos_sin_cache % 16 != 0 || (uintptr_t)k_cache % 8 != 0 ||
      (uintptr_t)v_cache % 8 != 0)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: tensors must be 16-byte aligned (caches 8) with a row stride of 8 elements",
                fn);
  nvamd::QkNormRopeParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qkv_stride = qkv_stride0;
  p.positions = positions;
  p.q_weight = static_cast<const uint16_t*>(q_norm_weight);
  p.k_weight = static_cast<const uint16_t*>(k_norm_weight);
  p.cos_sin = cos_sin_cache;
  p.max_position = max_position;
  p.slot_mapping = slot_mapping;
  p.k_cache = static_cast<uint8_t*>(k_cache);
  p.v_cache = static_cast<uint8_t*>(v_cache);
  p.num_slots = num_slots;
  p.q_out = static_cast<uint16_t*>(q_out);
  p.k_out = static_cast<uint16_t*>(k_out);
  p.num_tokens = num_tokens;
  p.Hq = num_heads;
  p.Hkv = num_kv_heads;
  p.eps = eps;
  return launch_status(nvamd::launch_qk_norm_rope_store(p, (hipStream_t)stream), fn);
}

int32_t nvamd_fp8_act_quant(const void* x, int64_t x_stride0, int32_t x_dtype, void* xq, void* x_scale, int64_t M,
                            int64_t K, void* stream) {
  static const char* fn = "fp8_act_quant";
  if (M < 0 || K <= 0 || K % 128 != 0 || x_stride0 < K)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: bad sizes (M=%lld K=%lld stride=%lld; K %% 128 == 0)", fn,
                (long long)M, (long long)K, (long long)x_stride0);
  if (x_dtype != NVAMD_DTYPE_BF16 && x_dtype != NVAMD_DTYPE_F16)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: x_dtype must be bf16 or fp16 (got %d)", fn, x_dtype);
  if (M == 0) return ok();
  if (M > 0x7fffffffll || K > 128ll * 16 * 0xffff)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: M=%lld K=%lld beyond the launch grid (M < 2^31, K < 2^27)", fn,
                (long long)M, (long long)K);
  if (!x || !xq || !x_scale) return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if ((uintptr_t)x % 16 != 0 || x_stride0 % 8 != 0 || (uintptr_t)xq % 8 != 0 || (uintptr_t)x_scale % 2 != 0)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: x must be 16-byte aligned with a row stride of 8 elements (xq 8-byte aligned)",
                fn);
  return launch_status(nvamd::launch_fp8_act_quant(x, x_stride0, x_dtype == NVAMD_DTYPE_F16, xq, x_scale, M, K,
                                                   (hipStream_t)stream),
                       fn);
}

namespace {

int64_t device_lds_limit() {
  int dev = 0, lds_limit = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&lds_limit, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lds_limit <= 0)
    lds_limit = 160 * 1024;
  return lds_limit;
}

}  // namespace

int64_t nvamd_fp8_block_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % 128 != 0 || K % 128 != 0 || N > 0x7fffffffll || K > 0x7fffffffll) return 0;
  return nvamd::fp8_skinny_workspace_bytes(M, N, (int)(K / 128), device_cu_count(), device_lds_limit());
}

int32_t nvamd_fp8_block_gemm(const void* xq, const void* x_scale, const void* weight, int64_t weight_stride0,
                             const void* weight_scale, void* out, int64_t out_stride0, int32_t out_dtype, int64_t M,
                             int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
  static const char* fn = "fp8_block_gemm";
  if (M < 0 || N <= 0 || K <= 0 || N % 128 != 0 || K % 128 != 0 || weight_stride0 < K || out_stride0 < N ||
      N > 0x7fffffffll || K > 0x7fffffffll)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: bad sizes (M=%lld N=%lld K=%lld; N, K multiples of 128)", fn,
                (long long)M, (long long)N, (long long)K);
  if (out_dtype != NVAMD_DTYPE_BF16 && out_dtype != NVAMD_DTYPE_F16)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: out_dtype must be bf16 or fp16 (got %d)", fn, out_dtype);
  if (M == 0) return ok();
  if (workspace_bytes < 0 || (workspace_bytes > 0 && workspace == nullptr))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: workspace_bytes=%lld with a null workspace", fn,
                (long long)workspace_bytes);
  if ((uintptr_t)workspace % 16 != 0)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: workspace must be 16-byte aligned", fn);
  if (!xq || !x_scale || !weight || !weight_scale || !out) return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if ((uintptr_t)xq % 16 != 0 || (uintptr_t)x_scale % 16 != 0 || (uintptr_t)weight % 16 != 0 ||
      weight_stride0 % 16 != 0 || (uintptr_t)weight_scale % 16 != 0 || (uintptr_t)out % 8 != 0 || out_stride0 % 4 != 0)
    return fail(NVAMD_ERR_UNSUPPORTED,
                "%s: operands must be 16-byte aligned (out 8), weight row stride a multiple of 16 bytes, out row stride "
                "a multiple of 4 elements",
                fn);
  if (weight_stride0 * 256 > 0xffffffffll || M * K > (1ll << 46))
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: weight row stride or activation size beyond 32-bit tile offsets", fn);
  const int64_t lds_limit = device_lds_limit();
  const int Kc = (int)(K / 128);
  const nvamd::SkinnyPlan plan = nvamd::fp8_skinny_plan(M, N, Kc, device_cu_count(), workspace_bytes, lds_limit);
  const int config = plan.cw > 0 ? 0 : nvamd::fp8_gemm_pick_config(M, N, Kc, device_cu_count(), lds_limit);
  if (config < 0)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: K=%lld needs more LDS for the tile scales than the device has", fn,
                (long long)K);
  nvamd::Fp8GemmParams p{};
  p.xq = static_cast<const uint8_t*>(xq);
  p.x_scale = static_cast<const uint16_t*>(x_scale);
  p.w = static_cast<const uint8_t*>(weight);
  p.w_scale = static_cast<const uint16_t*>(weight_scale);
  p.out = static_cast<uint16_t*>(out);
  p.w_stride = weight_stride0;
  p.out_stride = out_stride0;
  p.M = M;
  p.N = (int)N;
  p.K = (int)K;
  p.Kc = Kc;
  if (plan.cw > 0)
    return launch_status(nvamd::launch_fp8_skinny_gemm(p, plan, out_dtype == NVAMD_DTYPE_F16,
                                                       static_cast<float*>(workspace), (hipStream_t)stream),
                         fn);
  return launch_status(nvamd::launch_fp8_block_gemm(p, config, out_dtype == NVAMD_DTYPE_F16, (hipStream_t)stream), fn);
}

int32_t nvamd_build_attention_metadata(const int32_t* packed, int64_t packed_ints, int32_t num_seqs, int32_t num_plain,
                                       int32_t block_size,
                                       int64_t num_tokens, int64_t num_slots, int32_t num_table_rows,
                                       int32_t max_table_len, int64_t* positions, int32_t* slot_mapping,
                                       int32_t* context_lens, int32_t* cu_seqlens_q, int32_t* cu_seqlens_k,
                                       int32_t* block_tables, void* stream) {
  static const char* fn = "build_attention_metadata";
  if (num_seqs < 0 || num_seqs > nvamd::kMetaMaxSeqs || num_plain < 0 || num_plain > num_seqs || block_size <= 0 ||
      num_tokens < 0 || num_slots < 0 || num_table_rows < 0 || num_table_rows > num_seqs || max_table_len < 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT,
                "%s: bad sizes (seqs=%d of at most %d, plain=%d, block_size=%d, tokens=%lld, slots=%lld, rows=%d, "
                "width=%d)",
                fn, num_seqs, nvamd::kMetaMaxSeqs, num_plain, block_size, (long long)num_tokens, (long long)num_slots,
                num_table_rows, max_table_len);
  if (num_seqs == 0) return ok();
  if (packed_ints < 4ll * num_seqs)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: packed holds %lld ints, fewer than the %d descriptors", fn,
                (long long)packed_ints, num_seqs);
  const int n_var = num_seqs - num_plain;
  if (!packed || (num_tokens > 0 && !positions) || (num_slots > 0 && !slot_mapping) ||
      (num_plain > 0 && !context_lens) || (n_var > 0 && (!cu_seqlens_q || !cu_seqlens_k)) ||
      ((int64_t)num_table_rows * max_table_len > 0 && !block_tables))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if ((uintptr_t)packed % 16 != 0) return fail(NVAMD_ERR_UNSUPPORTED, "%s: packed must be 16-byte aligned", fn);
  nvamd::AttnMetaParams p{};
  p.packed = packed;
  p.packed_ints = packed_ints;
  p.num_seqs = num_seqs;
  p.num_plain = num_plain;
  p.block_size = block_size;
  p.max_table_len = max_table_len;
  p.cap_tokens = num_tokens;
  p.cap_slots = num_slots;
  p.cap_rows = num_table_rows;
  p.positions = positions;
  p.slot_mapping = slot_mapping;
  p.context_lens = context_lens;
  p.cu_seqlens_q = cu_seqlens_q;
  p.cu_seqlens_k = cu_seqlens_k;
  p.block_tables = block_tables;
  const int64_t units = num_tokens + (int64_t)num_table_rows * max_table_len + num_plain + (n_var > 0 ? n_var + 1 : 0);
  return launch_status(nvamd::launch_build_metadata(p, units, (hipStream_t)stream), fn);
}

// Workgroups per sampled row: about two per CU over the call, 1 .. 32.
static int64_t sample_parts(int64_t rows) {
  const int64_t cus = device_cu_count();
  return std::min<int64_t>(32, std::max<int64_t>(1, (2 * cus + rows - 1) / rows));
}

int32_t nvamd_select_logit_rows(const void* x, int64_t x_stride0, int64_t x_rows, int32_t hidden, int32_t elem_bytes,
                                const int32_t* cu_seqlens_q, int32_t num_plain, int32_t num_spec_seqs,
                                int32_t num_spec_rows, int32_t num_prefill_seqs, void* out, int64_t out_stride0,
                                void* stream) {
  static const char* fn = "select_logit_rows";
  if (x_rows < 0 || hidden <= 0 || (elem_bytes != 2 && elem_bytes != 4) || num_plain < 0 || num_spec_seqs < 0 ||
      num_spec_rows < 0 || num_prefill_seqs < 0 || x_stride0 < hidden || out_stride0 < hidden)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: bad sizes", fn);
  const int64_t out_rows = (int64_t)num_plain + num_spec_rows + num_prefill_seqs;
  if ((int64_t)num_plain + num_spec_rows > x_rows)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: %lld kept prefix rows exceed the %lld rows of x", fn,
                (long long)((int64_t)num_plain + num_spec_rows), (long long)x_rows);
  if (out_rows == 0) return ok();
  if (!x || !out || (num_prefill_seqs > 0 && !cu_seqlens_q)) return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  const int64_t row_bytes = (int64_t)hidden * elem_bytes;
  if (row_bytes % 16 != 0 || row_bytes > 0x7fffffff || (uintptr_t)x % 16 != 0 || (uintptr_t)out % 16 != 0 ||
      (x_stride0 * elem_bytes) % 16 != 0 || (out_stride0 * elem_bytes) % 16 != 0)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: rows must be whole 16-byte units, 16-byte aligned", fn);
  return launch_status(nvamd::launch_select_rows(x, x_stride0 * elem_bytes, x_rows, (int)row_bytes, cu_seqlens_q,
                                                 num_plain, num_spec_rows, num_spec_seqs, out_rows, out,
                                                 out_stride0 * elem_bytes, (hipStream_t)stream),
                       fn);
}

// Workspace of nvamd_sample: the noise path's per-part results (parts x rows
// x (fp32 score + int64 index)) or the in-kernel path's per-quad results
// (rows x quads x (fp32 score + int32 group)), whichever is larger.
static int64_t sample_workspace(int64_t rows, int64_t vocab) {
  const int64_t tasks = rows * nvamd::sample_quads(vocab);
  return std::max<int64_t>(sample_parts(rows) * rows * 16, 2 * ((tasks * 4 + 15) & ~15ll));
}

int64_t nvamd_sample_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || rows > 0x7fffffff || vocab <= 0 || vocab >= 0x7fffffff) return 0;
  return sample_workspace(rows, vocab);
}

int32_t nvamd_sample(const void* logits, int32_t logits_dtype, int64_t stride0, int64_t rows, int64_t vocab,
                     const float* temperatures, const float* noise, uint64_t seed, uint64_t offset, int64_t* out,
                     void* workspace, int64_t workspace_bytes, void* stream) {
  static const char* fn = "sample";
  if (rows < 0 || rows > 0x7fffffff || vocab <= 0 || stride0 < vocab || logits_dtype < NVAMD_LOGITS_BF16 ||
      logits_dtype > NVAMD_LOGITS_F32)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: bad sizes or dtype (rows=%lld vocab=%lld dtype=%d)", fn,
                (long long)rows, (long long)vocab, logits_dtype);
  if (vocab >= 0x7fffffff - 4096)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: vocabulary of %lld entries: at most 2^31 - 4098", fn, (long long)vocab);
  if (rows == 0) return ok();
  if (!logits || !temperatures || !out) return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  const int64_t need = sample_workspace(rows, vocab);
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 16 != 0)
    return fail(NVAMD_ERR_WORKSPACE, "%s: workspace of %lld bytes (16-byte aligned) needed", fn, (long long)need);
  char* ws = static_cast<char*>(workspace);
  if (noise == nullptr) {
    const int64_t tasks = rows * nvamd::sample_quads(vocab);
    float* task_score = reinterpret_cast<float*>(ws);
    int* task_group = reinterpret_cast<int*>(ws + ((tasks * 4 + 15) & ~15ll));
    return launch_status(nvamd::launch_sample_group(logits, logits_dtype, stride0, rows, vocab, temperatures, seed,
                                                    offset, out, task_score, task_group, (hipStream_t)stream),
                         fn);
  }
  const int parts = sample_parts(rows);
  float* part_score = reinterpret_cast<float*>(ws);
  int64_t* part_index = reinterpret_cast<int64_t*>(ws + ((parts * rows * 4 + 15) & ~15ll));
  return launch_status(nvamd::launch_sample_noise(logits, logits_dtype, stride0, rows, vocab, temperatures, noise,
                                                  out, part_score, part_index, (int)parts, (hipStream_t)stream),
                       fn);
}

int64_t nvamd_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                     int32_t max_num_blocks, int32_t block_size, int32_t part_tokens) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || max_num_blocks <= 0 || block_size <= 0)
    return 0;
  if (num_heads % num_kv_heads != 0) return 0;
  if (use_stream_k(batch, num_kv_heads, part_tokens))
    return stream_k_bytes(batch, num_kv_heads, num_heads / num_kv_heads, num_heads / num_kv_heads, false);
  const int64_t kv_cap = (int64_t)max_num_blocks * block_size;
  const int64_t part = choose_part_tokens((int64_t)batch * kv_head_groups(num_kv_heads), kv_cap,
                                          part_tokens, block_size);
  return partial_bytes(batch, num_heads, ceil_div(kv_cap, part));
}

}  // extern "C"

namespace {

// nvamd_fp8_decode_attention; with lib_scratch, the workspace is the
// library's scratch array (workspace / workspace_bytes are ignored).
int32_t decode_attention(const char* fn, void* out, const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_tables, const int32_t* context_lens, int32_t batch,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int64_t num_blocks,
                         int32_t block_size, int32_t max_num_blocks, float softmax_scale, int32_t part_tokens,
                         void* workspace, int64_t workspace_bytes, int32_t qo_dtype, void* stream,
                         bool lib_scratch) {
  if (int32_t e = check_heads(fn, num_heads, num_kv_heads, head_dim)) return e;
  if (int32_t e = check_qo_dtype(fn, qo_dtype)) return e;
  if (!(softmax_scale > 0.f) || !std::isfinite(softmax_scale))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: softmax_scale must be positive and finite", fn);
  if (batch < 0 || num_blocks < 0 || max_num_blocks < 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: negative size", fn);
  if (block_size <= 0 || block_size % 16 != 0)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: block_size must be a positive multiple of 16 (got %d)", fn, block_size);
  if (part_tokens < 0 || part_tokens % kPartAlign != 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: part_tokens must be 0 or a multiple of %d", fn, kPartAlign);
  if (part_tokens > max_part_tokens(block_size))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: part_tokens %d exceeds %lld (%lld blocks of %d)", fn,
                part_tokens, (long long)max_part_tokens(block_size), (long long)kMaxPartBlocks, block_size);
  const int G = num_heads / num_kv_heads;
  if (G > kMqMaxCols)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: more than %d query heads per kv head", fn, kMqMaxCols);
  if (batch == 0) return ok();
  if (max_num_blocks == 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: block_tables has no columns", fn);
  if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);

  if (lib_scratch) {
    const int64_t need = nvamd_decode_workspace_bytes(batch, num_heads, num_kv_heads, max_num_blocks, block_size,
                                                      part_tokens);
    if (need > NVAMD_NOALLOC_SCRATCH_BYTES)
      return fail(NVAMD_ERR_WORKSPACE, "%s: these shapes need %lld bytes of scratch, more than the %lld the library "
                  "holds", fn, (long long)need, (long long)NVAMD_NOALLOC_SCRATCH_BYTES);
    if (int32_t e = noalloc_scratch(fn, &workspace)) return e;
    workspace_bytes = NVAMD_NOALLOC_SCRATCH_BYTES;
  }

  nvamd::MqParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint8_t*>(k_cache);
  p.v = static_cast<const uint8_t*>(v_cache);
  p.block_tables = block_tables;
  p.bt_stride = max_num_blocks;
  p.context_lens = context_lens;
  p.cu_q = p.cu_k = nullptr;
  p.out = static_cast<uint16_t*>(out);
  p.q_rows = batch;
  p.kv_rows = num_blocks * block_size;
  p.num_seqs = batch;
  p.Hq = num_heads;
  p.Hkv = num_kv_heads;
  p.G = G;
  p.block_size = block_size;
  const int64_t kv_cap = (int64_t)max_num_blocks * block_size;
  p.mq_max_q = 1;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  p.out_f16 = qo_dtype == NVAMD_DTYPE_F16;
  const int ncb = (G + 15) / 16;
  if (use_stream_k(batch, num_kv_heads, part_tokens)) {
    const int64_t need = stream_k_bytes(batch, num_kv_heads, G, G, false);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(NVAMD_ERR_WORKSPACE, "%s: workspace of %lld bytes required (got %lld)", fn,
                  (long long)need, (long long)workspace_bytes);
    p.part_tokens = (int)std::min<int64_t>(kv_cap, 0x7fffffff);
    p.max_parts = 1;
    p.sk_heads = stream_k_heads(num_kv_heads, false);
    p.sk_wgs = stream_k_wgs(ncb, p.sk_heads, G, false);
    p.sk_cols = G;
    p.sk_prefix = static_cast<int32_t*>(workspace);
    p.sk_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + stream_k_prefix_bytes(batch));
    return launch_status(nvamd::launch_decode_sk(p, ncb, true, nullptr, nullptr, (hipStream_t)stream), fn);
  }
  const int64_t part = choose_part_tokens((int64_t)batch * kv_head_groups(num_kv_heads), kv_cap,
                                          part_tokens, block_size);
  p.part_tokens = (int)part;
  p.max_parts = (int)ceil_div(kv_cap, part);
  const int64_t need = partial_bytes(p.q_rows, p.Hq, p.max_parts);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(NVAMD_ERR_WORKSPACE, "%s: workspace of %lld bytes required (got %lld)", fn,
                (long long)need, (long long)workspace_bytes);
  set_partials(p, need > 0 ? workspace : nullptr);
  return launch_status(nvamd::launch_paged_mq(p, ncb, (hipStream_t)stream), fn);
}

}  // namespace

extern "C" {

int32_t nvamd_fp8_decode_attention(void* out, const void* q, const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, const int32_t* context_lens,
                                   int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int64_t num_blocks, int32_t block_size,
                                   int32_t max_num_blocks, float softmax_scale, int32_t part_tokens,
                                   void* workspace, int64_t workspace_bytes, int32_t qo_dtype, void* stream) {
  return decode_attention("fp8_decode_attention", out, q, k_cache, v_cache, block_tables, context_lens, batch,
                          num_heads, num_kv_heads, head_dim, num_blocks, block_size, max_num_blocks, softmax_scale,
                          part_tokens, workspace, workspace_bytes, qo_dtype, stream, false);
}

int32_t nvamd_fp8_decode_attention_noalloc(void* out, const void* q, const void* k_cache, const void* v_cache,
                                           const int32_t* block_tables, const int32_t* context_lens,
                                           int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                           int32_t head_dim, int64_t num_blocks, int32_t block_size,
                                           int32_t max_num_blocks, float softmax_scale, int32_t qo_dtype,
                                           void* stream) {
  return decode_attention("fp8_decode_attention_noalloc", out, q, k_cache, v_cache, block_tables, context_lens,
                          batch, num_heads, num_kv_heads, head_dim, num_blocks, block_size, max_num_blocks,
                          softmax_scale, 0, nullptr, 0, qo_dtype, stream, true);
}

int64_t nvamd_prefill_workspace_bytes(int64_t num_tokens, int32_t num_seqs, int32_t num_heads,
                                      int32_t num_kv_heads, int64_t kv_cap, int32_t max_seqlen_q,
                                      int32_t block_size, int32_t part_tokens) {
  if (num_tokens <= 0 || num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || kv_cap <= 0) return 0;
  const int G = num_heads / num_kv_heads;
  if (G <= 0 || G > kMqMaxCols) return 0;
  const int64_t part = choose_part_tokens((int64_t)num_seqs * kv_head_groups(num_kv_heads), kv_cap,
                                          part_tokens, block_size);
  int64_t partials = partial_bytes(num_tokens, num_heads, ceil_div(kv_cap, part));
  if (block_size > 0 && use_stream_k(num_seqs, num_kv_heads, part_tokens))  // paged: the balanced kernel
    partials = stream_k_bytes(num_seqs, num_kv_heads, G, short_cols(G, max_seqlen_q), true);
  return align_up(partials) + prefill_layout(num_seqs, num_kv_heads, G, max_seqlen_q).bytes();
}

int32_t nvamd_fp8_prefill_attention(void* out, const void* q, const void* k, const void* v,
                                    const int32_t* block_tables, const int32_t* cu_seqlens_q,
                                    const int32_t* cu_seqlens_k, int64_t num_tokens, int32_t num_seqs,
                                    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int64_t num_kv_rows, int32_t block_size, int32_t max_num_blocks,
                                    int32_t max_seqlen_q, int32_t max_seqlen_k, float softmax_scale,
                                    int32_t part_tokens, void* workspace, int64_t workspace_bytes,
                                    int32_t qo_dtype, void* stream) {
  static const char* fn = "fp8_prefill_attention";
  (void)max_seqlen_k;
  if (int32_t e = check_heads(fn, num_heads, num_kv_heads, head_dim)) return e;
  if (int32_t e = check_qo_dtype(fn, qo_dtype)) return e;
  if (!(softmax_scale > 0.f) || !std::isfinite(softmax_scale))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: softmax_scale must be positive and finite", fn);
  if (num_tokens < 0 || num_seqs < 0 || num_kv_rows < 0 || max_seqlen_q < 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: negative size", fn);
  const bool paged = block_tables != nullptr;
  if (paged && (block_size <= 0 || block_size % 16 != 0))
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: block_size must be a positive multiple of 16 (got %d)", fn, block_size);
  if (paged && max_num_blocks <= 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: block_tables has no columns", fn);
  // the prefill kernel finds a key's block by a reciprocal multiply, exact
  // below 2^35 / block_size keys per sequence
  if (paged && (int64_t)max_num_blocks * block_size >= (1ll << 35) / block_size)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: %d blocks of %d tokens per sequence exceed the addressable keys", fn,
                max_num_blocks, block_size);
  if (part_tokens < 0 || part_tokens % kPartAlign != 0)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: part_tokens must be 0 or a multiple of %d", fn, kPartAlign);
  if (paged && part_tokens > max_part_tokens(block_size))
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: part_tokens %d exceeds %lld (%lld blocks of %d)", fn,
                part_tokens, (long long)max_part_tokens(block_size), (long long)kMaxPartBlocks, block_size);
  const int G = num_heads / num_kv_heads;
  if (G > kMqMaxCols)
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: more than %d query heads per kv head", fn, kMqMaxCols);
  if (num_tokens == 0 || num_seqs == 0 || max_seqlen_q == 0) return ok();
  if (!out || !q || !k || !v || !cu_seqlens_q || !cu_seqlens_k)
    return fail(NVAMD_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);

  const int mq_max_q = kMqMaxCols / G;
  const int64_t kv_cap = paged ? (int64_t)max_num_blocks * block_size : std::max<int64_t>(num_kv_rows, 1);
  const int64_t part = choose_part_tokens((int64_t)num_seqs * kv_head_groups(num_kv_heads), kv_cap,
                                          part_tokens, paged ? block_size : 0);
  // Short-query rows of a paged call take the balanced (stream-K) kernel
  // when decode would; otherwise the split-KV kernel.
  const bool sk = paged && use_stream_k(num_seqs, num_kv_heads, part_tokens);
  const int64_t partials = sk ? stream_k_bytes(num_seqs, num_kv_heads, G, short_cols(G, max_seqlen_q), true)
                              : partial_bytes(num_tokens, num_heads, ceil_div(kv_cap, part));
  const PrefillLayout layout = prefill_layout(num_seqs, num_kv_heads, G, max_seqlen_q);
  const int64_t need = align_up(partials) + layout.bytes();
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(NVAMD_ERR_WORKSPACE, "%s: workspace of %lld bytes required (got %lld)", fn,
                (long long)need, (long long)workspace_bytes);

  // Short-query sequences: split-KV multi-query kernel.
  nvamd::MqParams mp{};
  mp.q = static_cast<const uint16_t*>(q);
  mp.k = static_cast<const uint8_t*>(k);
  mp.v = static_cast<const uint8_t*>(v);
  mp.block_tables = block_tables;
  mp.bt_stride = paged ? max_num_blocks : 0;
  mp.context_lens = nullptr;
  mp.cu_q = cu_seqlens_q;
  mp.cu_k = cu_seqlens_k;
  mp.out = static_cast<uint16_t*>(out);
  mp.q_rows = num_tokens;
  mp.kv_rows = num_kv_rows;
  mp.num_seqs = num_seqs;
  mp.Hq = num_heads;
  mp.Hkv = num_kv_heads;
  mp.G = G;
  mp.block_size = paged ? block_size : 64;
  mp.part_tokens = (int)part;
  mp.max_parts = (int)ceil_div(kv_cap, part);
  mp.mq_max_q = std::min(mq_max_q, max_seqlen_q);
  mp.scale_log2 = softmax_scale * 1.4426950408889634f;
  mp.out_f16 = qo_dtype == NVAMD_DTYPE_F16;
  const int ncb = (G * mp.mq_max_q + 15) / 16;
  const bool all_short = max_seqlen_q <= mq_max_q;
  if (sk) {
    mp.part_tokens = (int)std::min<int64_t>(kv_cap, 0x7fffffff);
    mp.max_parts = 1;
    mp.sk_heads = stream_k_heads(num_kv_heads, true);
    mp.sk_wgs = stream_k_wgs(ncb, mp.sk_heads, G, true);
    mp.sk_cols = short_cols(G, max_seqlen_q);
    mp.sk_prefix = static_cast<int32_t*>(workspace);
    mp.sk_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + stream_k_prefix_bytes(num_seqs));
    // balanced pass over the short-query rows (sequences with longer query
    // runs take no stages and are left alone); its merge is a launch of its
    // own when every sequence is short
    if (all_short)
      return launch_status(nvamd::launch_decode_sk(mp, ncb, true, nullptr, nullptr, (hipStream_t)stream), fn);
  } else {
    set_partials(mp, partials > 0 ? workspace : nullptr);
    if (max_seqlen_q <= mq_max_q)  // short sequences only: the split-KV kernel and its merge
      return launch_status(nvamd::launch_paged_mq(mp, ncb, (hipStream_t)stream), fn);
  }

  // Longer sequences: MFMA prefill kernel.  Two launches: the short-query
  // pass (which also writes the prefill work list), then the prefill kernel
  // (which also merges the short-query partitions).
  nvamd::PrefillParams pp{};
  pp.q = static_cast<const uint16_t*>(q);
  pp.k = static_cast<const uint8_t*>(k);
  pp.v = static_cast<const uint8_t*>(v);
  pp.block_tables = block_tables;
  pp.bt_stride = paged ? max_num_blocks : 0;
  pp.cu_q = cu_seqlens_q;
  pp.cu_k = cu_seqlens_k;
  pp.out = static_cast<uint16_t*>(out);
  pp.q_rows = num_tokens;
  pp.kv_rows = num_kv_rows;
  pp.num_seqs = num_seqs;
  pp.Hq = num_heads;
  pp.Hkv = num_kv_heads;
  pp.G = G;
  pp.GW = heads_per_workgroup(G);
  pp.BM = prefill_bm(G);
  pp.n_hgroups = G / pp.GW;
  pp.n_mblocks = (int)ceil_div(max_seqlen_q, pp.BM);
  pp.block_size = paged ? block_size : 64;
  pp.blk_magic = (uint32_t)(((1u << 31) - 1u) / (uint32_t)(pp.block_size / 16) + 1u);
  pp.mq_max_q = mq_max_q;
  pp.scale_log2 = softmax_scale * 1.4426950408889634f;
  pp.out_f16 = qo_dtype == NVAMD_DTYPE_F16;
  char* schedule = static_cast<char*>(workspace) + align_up(partials);
  if (layout.records > 0x7fffffff / ((int64_t)num_kv_heads * pp.n_hgroups))
    return fail(NVAMD_ERR_UNSUPPORTED, "%s: too many prefill work items", fn);
  pp.n_records = (int)layout.records;
  pp.slots_per_group = (int)layout.slots_per_group;
  pp.counters = reinterpret_cast<int*>(schedule + layout.list_bytes);
  pp.part = reinterpret_cast<uint32_t*>(schedule + layout.list_bytes + layout.counter_bytes);
  // The first launch is the short-query pass with one more workgroup that
  // writes the work list: the balanced kernel (one stream-K workgroup fewer,
  // so that the work-list workgroup is resident beside the others) or the
  // split-KV kernel.  The prefill kernel then merges either pass's partials.
  hipError_t e;
  if (sk) {
    mp.sk_wgs = std::max(mp.sk_wgs - 1, 1);
    e = nvamd::launch_decode_sk(mp, ncb, false, &pp, schedule, (hipStream_t)stream);
  } else {
    e = nvamd::launch_prefill_short(mp, ncb, pp, schedule, (hipStream_t)stream);
  }
  if (e != hipSuccess) return launch_status(e, fn);
  e = nvamd::launch_varlen_prefill(pp, schedule, mp, sk || mp.max_parts > 1, (hipStream_t)stream);
  if (e != hipSuccess) return launch_status(e, fn);
  return ok();
}

}  // extern "C"
