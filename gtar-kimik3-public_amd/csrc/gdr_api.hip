// C-ABI entry points of libgdr.so: argument validation, error reporting and dispatch to the kernel launchers.
// Nothing here allocates device memory; every launch goes to the caller's stream.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <string>

#include "gdr_internal.h"

// Device scratch of gdr_chunk_fwd_noalloc: the chunk path's workspace for callers that cannot allocate.  Each GPU the
// library runs on holds its own copy from the first such call until the process ends.  In host code `scratch`
// names a host-side stand-in, never the device array: kernels get the per-device address that
// hipGetSymbolAddress returns (scratch_on_device below).
static __device__ __align__(256) unsigned char scratch[GDR_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

bool valid_dtype(int d) { return d == GDR_F32 || d == GDR_BF16 || d == GDR_F16; }
int elem_size(int d) { return d == GDR_F32 ? 4 : 2; }

int check_view(const gdr_tensor& t, const char* name, bool required, bool f32_only) {
  if (!t.ptr) return required ? fail(GDR_ERR_INVALID, "%s: null pointer", name) : GDR_OK;
  if (!valid_dtype(t.dtype)) return fail(GDR_ERR_INVALID, "%s: unknown dtype code %d", name, t.dtype);
  if (f32_only && t.dtype != GDR_F32) return fail(GDR_ERR_INVALID, "%s: must be float32", name);
  if (t.stride_b < 0 || t.stride_h < 0 || t.stride_t < 0)
    return fail(GDR_ERR_INVALID, "%s: negative strides are not supported", name);
  return GDR_OK;
}

// Whether a chunk-mode call runs the sequential path -- the recurrent kernel over every token of each sequence, the
// state, every product and every sum in fp32 -- instead of the chunk kernels: q, k, v all fp32 (the reference's
// kernels take fp32 dot operands for fp32 inputs, src/ops/kimi_delta_attention.py:99-100, :130), or a key dim the
// chunk kernels are not built for (they take 64 and 128; the reference's take any multiple of 64).
bool chunk_sequential(const gdr_args* a) {
  const bool f32 = a->q.dtype == GDR_F32 && a->k.dtype == GDR_F32 && a->v.dtype == GDR_F32;
  return f32 || (a->key_dim != 64 && a->key_dim != 128);
}

// The chunk backward's shapes: the chunk kernels' key dims (64, 128) and value dims (multiples of 64).
int check_bwd_shape(const gdr_args* a) {
  if (a->key_dim != 64 && a->key_dim != 128)
    return fail(GDR_ERR_UNSUPPORTED, "the chunk backward takes key dims 64 and 128 (got %d)", a->key_dim);
  if (a->value_dim % 64)
    return fail(GDR_ERR_UNSUPPORTED, "the chunk backward takes value dims that are multiples of 64 (got %d)",
                a->value_dim);
  return GDR_OK;
}

// Sizes, variant, head dims and varlen fields: everything that shapes the work, no pointer dereferenced.
int check_shape(const gdr_args* a, bool chunk) {
  if (!a) return fail(GDR_ERR_INVALID, "args is NULL");
  if (a->abi_version != GDR_ABI_VERSION)
    return fail(GDR_ERR_INVALID, "abi_version %d, library implements %d", a->abi_version, GDR_ABI_VERSION);
  if (a->variant < GDR_KDA || a->variant > GDR_DELTANET)
    return fail(GDR_ERR_INVALID, "unknown variant %d", a->variant);
  if (a->batch < 1 || a->heads < 1 || a->seq_len < 0)
    return fail(GDR_ERR_INVALID, "bad sizes B=%d H=%d T=%d", a->batch, a->heads, a->seq_len);
  // The recurrent kernel takes key dims 32, 64, 128, 192 and 256 (the powers of two the reference's recurrent kernel
  // takes up to 256, and the multiples of 64 its chunk kernels take up to 256); the chunk kernels take 64 and 128.
  const int K = a->key_dim;
  if (K != 32 && K != 64 && K != 128 && K != 192 && K != 256)
    return fail(GDR_ERR_UNSUPPORTED, "key dim %d not supported (32, 64, 128, 192 or 256)", K);
  const int vmul = chunk && !chunk_sequential(a) ? 64 : 32;
  if (a->value_dim < vmul || a->value_dim % vmul != 0 || a->value_dim > 1024)
    return fail(GDR_ERR_UNSUPPORTED, "value dim %d not supported (a multiple of %d up to 1024)", a->value_dim,
                vmul);
  if (a->cu_seqlens) {
    if (!chunk) return fail(GDR_ERR_INVALID, "cu_seqlens is only accepted by the chunk mode");
    if (a->batch != 1) return fail(GDR_ERR_INVALID, "cu_seqlens requires batch == 1 (got %d)", a->batch);
    if (a->n_seqs < 1) return fail(GDR_ERR_INVALID, "cu_seqlens given with n_seqs=%d", a->n_seqs);
  }
  return GDR_OK;
}

// gate_in_memory false: the fused prologue computes the gate, so args->gate must be NULL.
int check_common(const gdr_args* a, bool chunk, bool need_out = true, bool gate_in_memory = true) {
  int rc = check_shape(a, chunk);
  if (rc) return rc;
  const bool has_gate = a->variant != GDR_DELTANET && gate_in_memory;
  const bool has_beta = a->variant != GDR_GLA;
  if ((rc = check_view(a->q, "query", true, false))) return rc;
  if ((rc = check_view(a->k, "key", true, false))) return rc;
  if ((rc = check_view(a->v, "value", true, false))) return rc;
  if ((rc = check_view(a->out, "out", need_out, false))) return rc;
  if ((rc = check_view(a->gate, "gate", has_gate, true))) return rc;
  if ((rc = check_view(a->beta, "beta", has_beta, true))) return rc;
  if (!has_gate && a->gate.ptr)
    return fail(GDR_ERR_INVALID, gate_in_memory ? "DeltaNet takes no gate" : "gate must be NULL: it is computed");
  if (!has_beta && a->beta.ptr) return fail(GDR_ERR_INVALID, "GLA takes no beta");
  if ((reinterpret_cast<uintptr_t>(a->h0) | reinterpret_cast<uintptr_t>(a->ht)) % 16 != 0)
    return fail(GDR_ERR_INVALID, "initial/final state must be 16-byte aligned");
  return GDR_OK;
}

int check_rows16(const gdr_tensor& t, const char* name) {
  const int es = elem_size(t.dtype);
  if (reinterpret_cast<uintptr_t>(t.ptr) % 16 || (t.stride_b * es) % 16 || (t.stride_h * es) % 16 ||
      (t.stride_t * es) % 16)
    return fail(GDR_ERR_INVALID, "%s: base pointer and b/h/t strides must be 16-byte aligned", name);
  return GDR_OK;
}

// The prologue of gdr_chunk_fwd_fused (no pointer dereferenced).
int check_prologue(const gdr_args* a, const gdr_prologue* pro) {
  if (pro->flags & ~(GDR_PRO_NORM_QK | GDR_PRO_BETA_LOGITS | GDR_PRO_GATE_LOWRANK | GDR_PRO_CONV))
    return fail(GDR_ERR_INVALID, "unknown prologue flags 0x%x", pro->flags);
  if ((pro->flags & GDR_PRO_BETA_LOGITS) && a->variant == GDR_GLA)
    return fail(GDR_ERR_INVALID, "GLA takes no beta (GDR_PRO_BETA_LOGITS)");
  if (pro->flags & GDR_PRO_CONV) {
    if (pro->conv_size < 2 || pro->conv_size > 8)
      return fail(GDR_ERR_UNSUPPORTED, "in-kernel convolution of width %d not supported (2 to 8)", pro->conv_size);
    const char* names[] = {"q", "k", "v"};
    for (int i = 0; i < 3; ++i) {
      if (!pro->conv_weight[i] || reinterpret_cast<uintptr_t>(pro->conv_weight[i]) % 16)
        return fail(GDR_ERR_INVALID, "conv_weight[%d] (%s): null or not 16-byte aligned", i, names[i]);
      if (pro->conv_state_out[i] && pro->conv_state_out[i] == pro->conv_state_in[i])
        return fail(GDR_ERR_INVALID, "conv_state_out[%d] must not alias conv_state_in[%d]", i, i);
    }
  }
  if (!(pro->flags & GDR_PRO_GATE_LOWRANK)) return GDR_OK;
  if (a->variant != GDR_KDA && a->variant != GDR_GLA)
    return fail(GDR_ERR_UNSUPPORTED, "the low-rank gate is for the per-channel gates (KDA, GLA)");
  if (pro->rank < 32 || pro->rank > 512 || pro->rank % 32)
    return fail(GDR_ERR_UNSUPPORTED, "gate rank %d not supported (a multiple of 32 up to 512)", pro->rank);
  int rc = check_view(pro->gate_lowrank, "gate_lowrank", true, false);
  if (rc) return rc;
  if (pro->gate_lowrank.dtype != GDR_BF16) return fail(GDR_ERR_UNSUPPORTED, "gate_lowrank must be bf16");
  if (reinterpret_cast<uintptr_t>(pro->gate_lowrank.ptr) % 16 || (pro->gate_lowrank.stride_b * 2) % 16 ||
      (pro->gate_lowrank.stride_t * 2) % 16)
    return fail(GDR_ERR_INVALID, "gate_lowrank: base pointer and b/t strides must be 16-byte aligned");
  if (!pro->gate_weight || reinterpret_cast<uintptr_t>(pro->gate_weight) % 16)
    return fail(GDR_ERR_INVALID, "gate_weight: null or not 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(pro->gate_bias) % 16)
    return fail(GDR_ERR_INVALID, "gate_bias must be 16-byte aligned");
  if (!pro->a_log) return fail(GDR_ERR_INVALID, "a_log: null pointer");
  return GDR_OK;
}

// Address of `scratch` on `device`, looked up once per device (with that device current) and kept.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

hipError_t scratch_on_device(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = g_scratch_ptr[device].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[device].load(std::memory_order_relaxed);
    if (!p) {
      int current = -1;
      hipError_t e = hipGetDevice(&current);
      if (e != hipSuccess) return e;
      if (current != device && (e = hipSetDevice(device)) != hipSuccess) return e;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      const hipError_t restore = current != device ? hipSetDevice(current) : hipSuccess;
      if (e != hipSuccess) return e;
      if (restore != hipSuccess) return restore;
      if (!p) return hipErrorInvalidSymbol;
      g_scratch_ptr[device].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return hipSuccess;
}

// The chunk op on the sequential path (chunk_sequential): q, k, v of one dtype, bf16 or f32, read by the recurrent
// kernel one token at a time, packed sequences included; no workspace is used.
int chunk_fwd_sequential(const gdr_args* a, const gdr_prologue* pro, hipStream_t stream) {
  if (pro) return fail(GDR_ERR_UNSUPPORTED, "the fused prologue runs on the chunk kernels: key dims 64 and 128, bf16 q, "
                       "k, v (got key dim %d, dtype codes %d, %d, %d)", a->key_dim, a->q.dtype, a->k.dtype, a->v.dtype);
  int rc = check_common(a, true);
  if (rc) return rc;
  if (a->q.dtype != a->k.dtype || a->q.dtype != a->v.dtype || a->q.dtype == GDR_F16)
    return fail(GDR_ERR_UNSUPPORTED, "key dim %d runs the recurrent kernel, which reads q, k, v of one dtype, bf16 or f32 "
                "(got dtype codes %d, %d, %d)", a->key_dim, a->q.dtype, a->k.dtype, a->v.dtype);
  hipError_t e = gdr::launch_recurrent(*a, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "recurrent launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int chunk_fwd(const gdr_args* a, const gdr_prologue* pro, hipStream_t stream) {
  int rc = check_shape(a, true);
  if (rc) return rc;
  if (chunk_sequential(a)) return chunk_fwd_sequential(a, pro, stream);
  if (pro && (rc = check_prologue(a, pro))) return rc;
  const bool lowrank = pro && (pro->flags & GDR_PRO_GATE_LOWRANK);
  if ((rc = check_common(a, true, true, !lowrank))) return rc;
  if (pro && !a->workspace) return fail(GDR_ERR_INVALID, "the fused prologue needs a workspace (two-launch path)");
  // q, k, v are the MFMA operands' type: all bf16, or all f16 (the two-launch path of the plain op).
  const bool f16 = a->q.dtype == GDR_F16 && a->k.dtype == GDR_F16 && a->v.dtype == GDR_F16;
  if (!f16 && (a->q.dtype != GDR_BF16 || a->k.dtype != GDR_BF16 || a->v.dtype != GDR_BF16))
    return fail(GDR_ERR_UNSUPPORTED, "chunk mode reads q, k, v of one 16-bit type, bf16 or f16 (got dtype codes %d, "
                "%d, %d); the recurrent mode takes f32", a->q.dtype, a->k.dtype, a->v.dtype);
  if (f16 && (pro || !a->workspace))
    return fail(GDR_ERR_UNSUPPORTED, "f16 q, k, v run on the two-launch path of the plain op only (a workspace, no "
                "fused prologue)");
  // Rows of q, k, v, gate and out are moved with 16-byte accesses.
  const gdr_tensor* rows[] = {&a->q, &a->k, &a->v, &a->out, &a->gate};
  const char* names[] = {"query", "key", "value", "out", "gate"};
  for (int i = 0; i < 5; ++i) {
    const gdr_tensor& t = *rows[i];
    if (!t.ptr) continue;
    if (i == 4 && a->variant == GDR_GDN) continue;  // scalar gate: element access
    const int es = elem_size(t.dtype);
    if (reinterpret_cast<uintptr_t>(t.ptr) % 16 || (t.stride_b * es) % 16 || (t.stride_h * es) % 16 ||
        (t.stride_t * es) % 16)
      return fail(GDR_ERR_INVALID, "%s: base pointer and b/h/t strides must be 16-byte aligned", names[i]);
  }
  const int64_t need = gdr::chunk_workspace_bytes(*a);
  hipError_t e;
  if (a->workspace) {
    if (a->workspace_bytes < need)
      return fail(GDR_ERR_INVALID, "workspace of %lld bytes given, %lld required", (long long)a->workspace_bytes,
                  (long long)need);
    if (reinterpret_cast<uintptr_t>(a->workspace) % 256)
      return fail(GDR_ERR_INVALID, "workspace must be 256-byte aligned");
    e = gdr::launch_chunk_split(*a, pro ? *pro : gdr_prologue{}, stream);
  } else {
    e = gdr::launch_chunk(*a, stream);
  }
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "chunk launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

// Arguments of the chunk backward (both entry points) and its workspace.
int check_bwd(const gdr_args* a, const gdr_grads* g, void* workspace, int64_t workspace_bytes) {
  int rc = check_common(a, true, false);
  if (rc) return rc;
  if (!g) return fail(GDR_ERR_INVALID, "grads is NULL");
  if (a->cu_seqlens) return fail(GDR_ERR_UNSUPPORTED, "the chunk backward does not take packed varlen input");
  if ((rc = check_bwd_shape(a))) return rc;
  if (a->q.dtype != GDR_BF16 || a->k.dtype != GDR_BF16 || a->v.dtype != GDR_BF16)
    return fail(GDR_ERR_UNSUPPORTED, "the chunk backward reads bf16 q, k, v (got dtype codes %d, %d, %d)", a->q.dtype,
                a->k.dtype, a->v.dtype);
  const bool has_gate = a->variant != GDR_DELTANET, has_beta = a->variant != GDR_GLA;
  if ((rc = check_view(g->d_out, "d_out", true, false))) return rc;
  if (g->d_out.dtype != GDR_BF16) return fail(GDR_ERR_UNSUPPORTED, "d_out must be bf16 (the MFMA operand type)");
  if ((rc = check_view(g->d_query, "d_query", true, false))) return rc;
  if ((rc = check_view(g->d_key, "d_key", true, false))) return rc;
  if ((rc = check_view(g->d_value, "d_value", true, false))) return rc;
  const gdr_tensor* outs[] = {&g->d_query, &g->d_key, &g->d_value};
  const char* onames[] = {"d_query", "d_key", "d_value"};
  for (int i = 0; i < 3; ++i)
    if (outs[i]->dtype == GDR_F16) return fail(GDR_ERR_UNSUPPORTED, "%s: bf16 or f32 only", onames[i]);
  if ((rc = check_view(g->d_gate, "d_gate", has_gate, true))) return rc;
  if ((rc = check_view(g->d_beta, "d_beta", has_beta, true))) return rc;
  if (!has_gate && g->d_gate.ptr) return fail(GDR_ERR_INVALID, "DeltaNet has no gate gradient");
  if (!has_beta && g->d_beta.ptr) return fail(GDR_ERR_INVALID, "GLA has no beta gradient");
  if ((reinterpret_cast<uintptr_t>(g->d_final) | reinterpret_cast<uintptr_t>(g->d_initial)) % 16 != 0)
    return fail(GDR_ERR_INVALID, "d_final / d_initial must be 16-byte aligned");
  const gdr_tensor* rows[] = {&a->q, &a->k, &a->v, &a->gate, &g->d_out};
  const char* names[] = {"query", "key", "value", "gate", "d_out"};
  for (int i = 0; i < 5; ++i) {
    if (!rows[i]->ptr || (i == 3 && a->variant == GDR_GDN)) continue;
    if ((rc = check_rows16(*rows[i], names[i]))) return rc;
  }
  const gdr::BwdLayout L = gdr::chunk_bwd_layout(*a);
  if (!workspace) return fail(GDR_ERR_INVALID, "the chunk backward needs a workspace");
  if (workspace_bytes < L.total)
    return fail(GDR_ERR_INVALID, "workspace of %lld bytes given, %lld required", (long long)workspace_bytes,
                (long long)L.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(GDR_ERR_INVALID, "workspace must be 256-byte aligned");
  return GDR_OK;
}

}  // namespace

extern "C" {

int gdr_abi_version(void) { return GDR_ABI_VERSION; }

const char* gdr_last_error(void) { return g_last_error.c_str(); }

int gdr_recurrent_fwd(const gdr_args* a, hipStream_t stream) {
  int rc = check_common(a, false);
  if (rc) return rc;
  if (a->q.dtype != a->k.dtype || a->q.dtype != a->v.dtype || a->q.dtype == GDR_F16)
    return fail(GDR_ERR_UNSUPPORTED, "recurrent mode reads q, k, v of one dtype, bf16 or f32 (got dtype codes %d, %d, %d)",
                a->q.dtype, a->k.dtype, a->v.dtype);
  hipError_t e = gdr::launch_recurrent(*a, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "recurrent launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int gdr_recurrent_verify(const gdr_args* a, float* updates, hipStream_t stream) {
  int rc = check_common(a, false);
  if (rc) return rc;
  if (a->q.dtype != a->k.dtype || a->q.dtype != a->v.dtype || a->q.dtype == GDR_F16)
    return fail(GDR_ERR_UNSUPPORTED, "recurrent mode reads q, k, v of one dtype, bf16 or f32 (got dtype codes %d, %d, %d)",
                a->q.dtype, a->k.dtype, a->v.dtype);
  if (!updates) return fail(GDR_ERR_INVALID, "updates: null pointer");
  if (reinterpret_cast<uintptr_t>(updates) % 16) return fail(GDR_ERR_INVALID, "updates must be 16-byte aligned");
  hipError_t e = gdr::launch_verify(*a, updates, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "verify launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

namespace {

// The arguments of a commit: sizes, k, the gate, the state pointers and the record (no pointer dereferenced).
int check_commit(const gdr_args* a, const float* updates) {
  int rc = check_shape(a, false);
  if (rc) return rc;
  const bool has_gate = a->variant != GDR_DELTANET;
  if ((rc = check_view(a->k, "key", true, false))) return rc;
  if (a->k.dtype == GDR_F16) return fail(GDR_ERR_UNSUPPORTED, "key: bf16 or f32 only");
  if ((rc = check_view(a->gate, "gate", has_gate, true))) return rc;
  if (!has_gate && a->gate.ptr) return fail(GDR_ERR_INVALID, "DeltaNet takes no gate");
  if (!a->ht) return fail(GDR_ERR_INVALID, "ht: null pointer (the commit writes the state)");
  if (!updates) return fail(GDR_ERR_INVALID, "updates: null pointer");
  if ((reinterpret_cast<uintptr_t>(a->h0) | reinterpret_cast<uintptr_t>(a->ht) |
       reinterpret_cast<uintptr_t>(updates)) % 16 != 0)
    return fail(GDR_ERR_INVALID, "initial/final state and updates must be 16-byte aligned");
  return GDR_OK;
}

// Byte ranges [p, p + n) and [q, q + m) overlap.
bool overlaps(const void* p, size_t n, const void* q, size_t m) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(q);
  return n && m && a < b + m && b < a + n;
}

}  // namespace

int gdr_recurrent_commit(const gdr_args* a, const float* updates, const int32_t* accepted, hipStream_t stream) {
  int rc = check_commit(a, updates);
  if (rc) return rc;
  hipError_t e = gdr::launch_commit(*a, updates, accepted, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "commit launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int gdr_recurrent_commit_verify(const gdr_args* prev, const float* prev_updates, const int32_t* accepted,
                                const gdr_args* a, float* updates, hipStream_t stream) {
  int rc = check_commit(prev, prev_updates);
  if (rc) return rc;
  if ((rc = check_common(a, false))) return rc;
  if (a->q.dtype != a->k.dtype || a->q.dtype != a->v.dtype || a->q.dtype == GDR_F16)
    return fail(GDR_ERR_UNSUPPORTED, "recurrent mode reads q, k, v of one dtype, bf16 or f32 (got dtype codes %d, %d, %d)",
                a->q.dtype, a->k.dtype, a->v.dtype);
  if (prev->variant != a->variant || prev->batch != a->batch || prev->heads != a->heads ||
      prev->key_dim != a->key_dim || prev->value_dim != a->value_dim)
    return fail(GDR_ERR_INVALID, "the previous block and the new block differ in variant or sizes");
  if (prev->k.dtype != a->q.dtype)
    return fail(GDR_ERR_UNSUPPORTED, "the previous block's key dtype (%d) differs from the new block's (%d)",
                prev->k.dtype, a->q.dtype);
  if (a->h0 != prev->ht)
    return fail(GDR_ERR_INVALID, "the new block's initial state must be the committed state (args->h0 == prev->ht)");
  if (!updates) return fail(GDR_ERR_INVALID, "updates: null pointer");
  if (reinterpret_cast<uintptr_t>(updates) % 16) return fail(GDR_ERR_INVALID, "updates must be 16-byte aligned");
  const size_t rows = size_t(a->batch) * a->heads * a->value_dim * sizeof(float);
  const size_t state = size_t(a->batch) * a->heads * a->key_dim * a->value_dim * sizeof(float);
  if (overlaps(updates, rows * a->seq_len, prev_updates, rows * prev->seq_len))
    return fail(GDR_ERR_INVALID, "updates must not overlap the previous block's record");
  if (a->ht && overlaps(a->ht, state, prev->ht, state))
    return fail(GDR_ERR_INVALID, "the final state must not overlap the committed state");
  hipError_t e = gdr::launch_commit_verify(*prev, prev_updates, accepted, *a, updates, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "commit-verify launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

namespace {

// The forward's arguments (no pointer dereferenced); the views in `views` share q's 16-bit dtype, rows 16-byte aligned.
int check_attention(const gdr_attention_args* a, const gdr_tensor* const* views, const char* const* names, int nviews) {
  if (!a) return fail(GDR_ERR_INVALID, "args is NULL");
  if (a->abi_version != GDR_ABI_VERSION)
    return fail(GDR_ERR_INVALID, "abi_version %d, library implements %d", a->abi_version, GDR_ABI_VERSION);
  if (a->batch < 1 || a->heads < 1 || a->kv_heads < 1 || a->seq_len < 0)
    return fail(GDR_ERR_INVALID, "bad sizes B=%d H=%d Hkv=%d T=%d", a->batch, a->heads, a->kv_heads, a->seq_len);
  if (a->heads % a->kv_heads) return fail(GDR_ERR_INVALID, "kv_heads %d does not divide heads %d", a->kv_heads, a->heads);
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(GDR_ERR_UNSUPPORTED, "head dim %d not supported (64 or 128)", a->head_dim);
  if (a->cu_seqlens && (a->batch != 1 || a->n_seqs < 1))
    return fail(GDR_ERR_INVALID, "cu_seqlens requires batch == 1 and n_seqs >= 1");
  if (reinterpret_cast<uintptr_t>(a->lse) % 4) return fail(GDR_ERR_INVALID, "lse must be 4-byte aligned");
  int rc;
  for (int i = 0; i < nviews; ++i) {
    if ((rc = check_view(*views[i], names[i], true, false))) return rc;
    if (views[i]->dtype != a->q.dtype)
      return fail(GDR_ERR_UNSUPPORTED, "%s: q, k, v, out (and the gradients) share one dtype", names[i]);
    if ((rc = check_rows16(*views[i], names[i]))) return rc;
  }
  if (a->q.dtype == GDR_F32) return fail(GDR_ERR_UNSUPPORTED, "attention reads bf16 or f16 (the MFMA operand types)");
  return GDR_OK;
}

}  // namespace

int gdr_attention_fwd(const gdr_attention_args* a, hipStream_t stream) {
  const gdr_tensor* views[] = {a ? &a->q : nullptr, a ? &a->k : nullptr, a ? &a->v : nullptr, a ? &a->out : nullptr};
  const char* names[] = {"query", "key", "value", "out"};
  if (const int rc = check_attention(a, views, names, 4)) return rc;
  hipError_t e = gdr::launch_attention(*a, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "attention launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int gdr_attention_bwd(const gdr_attention_args* a, const gdr_attention_grads* g, hipStream_t stream) {
  if (!g) return fail(GDR_ERR_INVALID, "grads is NULL");
  if (g->abi_version != GDR_ABI_VERSION)
    return fail(GDR_ERR_INVALID, "grads abi_version %d, library implements %d", g->abi_version, GDR_ABI_VERSION);
  const gdr_tensor* views[] = {a ? &a->q : nullptr, a ? &a->k : nullptr, a ? &a->v : nullptr, a ? &a->out : nullptr,
                               &g->d_out, &g->d_q, &g->d_k, &g->d_v};
  const char* names[] = {"query", "key", "value", "out", "d_out", "d_q", "d_k", "d_v"};
  if (const int rc = check_attention(a, views, names, 8)) return rc;
  if (!a->lse) return fail(GDR_ERR_INVALID, "lse is NULL: the backward reads the forward's row log-sum-exp");
  if (!g->delta || reinterpret_cast<uintptr_t>(g->delta) % 4)
    return fail(GDR_ERR_INVALID, "delta must be a non-NULL, 4-byte aligned fp32 [B][H][T] buffer");
  hipError_t e = gdr::launch_attention_bwd(*a, *g, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "attention backward launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int gdr_short_conv_fwd(const gdr_conv_args* a, hipStream_t stream) {
  if (!a) return fail(GDR_ERR_INVALID, "args is NULL");
  if (a->abi_version != GDR_ABI_VERSION)
    return fail(GDR_ERR_INVALID, "abi_version %d, library implements %d", a->abi_version, GDR_ABI_VERSION);
  if (a->batch < 1 || a->seq_len < 0 || a->channels < 1)
    return fail(GDR_ERR_INVALID, "bad sizes B=%d T=%d C=%d", a->batch, a->seq_len, a->channels);
  if (a->kernel_size < 2 || a->kernel_size > 8)
    return fail(GDR_ERR_UNSUPPORTED, "kernel size %d not supported (2 to 8)", a->kernel_size);
  if (a->cu_seqlens && (a->batch != 1 || a->n_seqs < 1))
    return fail(GDR_ERR_INVALID, "cu_seqlens requires batch == 1 and n_seqs >= 1");
  if (a->seq_len == 0) {  // no token: nothing to compute and no state entry to write (x, out may be NULL)
    g_last_error.clear();
    return GDR_OK;
  }
  int rc;
  if ((rc = check_view(a->x, "x", true, false)) || (rc = check_view(a->out, "out", true, false))) return rc;
  if (a->out.dtype != a->x.dtype) return fail(GDR_ERR_UNSUPPORTED, "out must have x's dtype");
  const int vec = 16 / elem_size(a->x.dtype);
  if (a->channels % vec) return fail(GDR_ERR_UNSUPPORTED, "channels must be a multiple of %d", vec);
  const gdr_tensor* rows[] = {&a->x, &a->out};
  const char* names[] = {"x", "out"};
  for (int i = 0; i < 2; ++i) {
    const int es = elem_size(rows[i]->dtype);
    if (reinterpret_cast<uintptr_t>(rows[i]->ptr) % 16 || (rows[i]->stride_b * es) % 16 || (rows[i]->stride_t * es) % 16)
      return fail(GDR_ERR_INVALID, "%s: base pointer and b/t strides must be 16-byte aligned", names[i]);
  }
  if (!a->weight) return fail(GDR_ERR_INVALID, "weight: null pointer");
  if (a->state_out && a->state_out == a->state_in) return fail(GDR_ERR_INVALID, "state_out must not alias state_in");
  hipError_t e = gdr::launch_short_conv(*a, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "short convolution launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int gdr_norm_gate_fwd(const gdr_norm_gate_args* a, hipStream_t stream) {
  if (!a) return fail(GDR_ERR_INVALID, "args is NULL");
  if (a->abi_version != GDR_ABI_VERSION)
    return fail(GDR_ERR_INVALID, "abi_version %d, library implements %d", a->abi_version, GDR_ABI_VERSION);
  if (a->batch < 1 || a->seq_len < 0 || a->heads < 1)
    return fail(GDR_ERR_INVALID, "bad sizes B=%d T=%d H=%d", a->batch, a->seq_len, a->heads);
  if (a->value_dim < 64 || a->value_dim > 256 || a->value_dim % 64)
    return fail(GDR_ERR_UNSUPPORTED, "value dim %d not supported (64, 128, 192 or 256)", a->value_dim);
  if (int64_t(a->batch) * a->seq_len * a->heads >= (int64_t(1) << 31))
    return fail(GDR_ERR_UNSUPPORTED, "B * T * H must be below 2^31");
  if (!(a->eps >= 0.f)) return fail(GDR_ERR_INVALID, "eps must be >= 0");
  int rc;
  if ((rc = check_view(a->x, "x", true, false)) || (rc = check_view(a->gate, "gate", true, false)) ||
      (rc = check_view(a->out, "out", true, false)))
    return rc;
  if (a->gate.dtype != a->x.dtype) return fail(GDR_ERR_UNSUPPORTED, "gate must have x's dtype");
  if (a->weight_dtype != GDR_F32 && a->weight_dtype != a->x.dtype)
    return fail(GDR_ERR_UNSUPPORTED, "weight must be f32 or x's dtype");
  const int want_out = a->weight_dtype == GDR_F32 ? GDR_F32 : a->x.dtype;
  if (a->out.dtype != want_out) return fail(GDR_ERR_UNSUPPORTED, "out dtype must be %d (type promotion)", want_out);
  if (!a->weight) return fail(GDR_ERR_INVALID, "weight: null pointer");
  const gdr_tensor* views[] = {&a->x, &a->gate, &a->out};
  const char* names[] = {"x", "gate", "out"};
  for (int i = 0; i < 3; ++i) {
    const int es = elem_size(views[i]->dtype);
    if (reinterpret_cast<uintptr_t>(views[i]->ptr) % 16 || (views[i]->stride_b * es) % 16 ||
        (views[i]->stride_h * es) % 16 || (views[i]->stride_t * es) % 16)
      return fail(GDR_ERR_INVALID, "%s: base pointer and b/h/t strides must be 16-byte aligned", names[i]);
  }
  hipError_t e = gdr::launch_norm_gate(*a, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "norm-gate launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int64_t gdr_chunk_workspace_bytes(const gdr_args* a) {
  const int rc = check_shape(a, true);
  if (rc) return rc;
  g_last_error.clear();
  // Read from the sizes alone (no dtype): key dims the chunk kernels do not take run the sequential path, which needs
  // no workspace; so do fp32 calls, which ignore the one they are given.
  return (a->key_dim == 64 || a->key_dim == 128) ? gdr::chunk_workspace_bytes(*a) : 0;
}

int gdr_chunk_fwd(const gdr_args* a, hipStream_t stream) { return chunk_fwd(a, nullptr, stream); }

int gdr_chunk_fwd_noalloc(const gdr_args* a, hipStream_t stream) {
  int rc = check_shape(a, true);
  if (rc) return rc;
  if (a->workspace) return fail(GDR_ERR_INVALID, "gdr_chunk_fwd_noalloc: workspace must be NULL (the library's "
                                "device scratch is used)");
  if (chunk_sequential(a)) return chunk_fwd_sequential(a, nullptr, stream);  // no scratch needed
  const int64_t need = gdr::chunk_workspace_bytes(*a);
  if (need > GDR_NOALLOC_SCRATCH_BYTES)
    return fail(GDR_ERR_UNSUPPORTED, "gdr_chunk_fwd_noalloc: this call needs %lld bytes of scratch, above the "
                "library's fixed %lld (one record per 64-token chunk and head); use gdr_chunk_fwd with a workspace",
                (long long)need, (long long)GDR_NOALLOC_SCRATCH_BYTES);
  int device = -1;
  hipError_t e = hipStreamGetDevice(stream, &device);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "gdr_chunk_fwd_noalloc: stream device: %s", hipGetErrorString(e));
  void* ptr = nullptr;
  if ((e = scratch_on_device(device, &ptr)) != hipSuccess)
    return fail(GDR_ERR_HIP, "gdr_chunk_fwd_noalloc: scratch address on device %d: %s", device, hipGetErrorString(e));
  gdr_args b = *a;
  b.workspace = ptr;
  b.workspace_bytes = GDR_NOALLOC_SCRATCH_BYTES;
  return chunk_fwd(&b, nullptr, stream);
}

int gdr_chunk_fwd_fused(const gdr_args* a, const gdr_prologue* pro, hipStream_t stream) {
  if (!pro) return fail(GDR_ERR_INVALID, "prologue is NULL");
  return chunk_fwd(a, pro, stream);
}

int64_t gdr_chunk_bwd_workspace_bytes(const gdr_args* a) {
  int rc = check_shape(a, true);
  if (rc) return rc;
  if (a->cu_seqlens) return fail(GDR_ERR_UNSUPPORTED, "the chunk backward does not take packed varlen input");
  if ((rc = check_bwd_shape(a))) return rc;
  g_last_error.clear();
  return gdr::chunk_bwd_layout(*a).total;
}

int gdr_chunk_bwd(const gdr_args* a, const gdr_grads* g, void* workspace, int64_t workspace_bytes,
                  hipStream_t stream) {
  const int rc = check_bwd(a, g, workspace, workspace_bytes);
  if (rc) return rc;
  const gdr::BwdLayout L = gdr::chunk_bwd_layout(*a);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  hipError_t e = gdr::launch_chunk_states(*a, L, ws, stream);
  if (e == hipSuccess) e = gdr::launch_chunk_bwd(*a, *g, L, ws, stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "chunk backward launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int gdr_chunk_fwd_train(const gdr_args* a, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  int rc = check_common(a, true, true);
  if (rc) return rc;
  if (a->cu_seqlens) return fail(GDR_ERR_UNSUPPORTED, "the chunk backward does not take packed varlen input");
  if ((rc = check_bwd_shape(a))) return rc;
  if (a->q.dtype != GDR_BF16 || a->k.dtype != GDR_BF16 || a->v.dtype != GDR_BF16)
    return fail(GDR_ERR_UNSUPPORTED, "the chunk backward reads bf16 q, k, v (got dtype codes %d, %d, %d)", a->q.dtype,
                a->k.dtype, a->v.dtype);
  if (a->out.dtype != GDR_BF16 && a->out.dtype != GDR_F32)
    return fail(GDR_ERR_UNSUPPORTED, "out: bf16 or f32 only");
  if (a->workspace)
    return fail(GDR_ERR_INVALID, "gdr_chunk_fwd_train: args->workspace must be NULL (the records go into the "
                "backward workspace)");
  const gdr_tensor* rows[] = {&a->q, &a->k, &a->v, &a->out, &a->gate};
  const char* names[] = {"query", "key", "value", "out", "gate"};
  for (int i = 0; i < 5; ++i) {
    if (!rows[i]->ptr || (i == 4 && a->variant == GDR_GDN)) continue;
    if ((rc = check_rows16(*rows[i], names[i]))) return rc;
  }
  const gdr::BwdLayout L = gdr::chunk_bwd_layout(*a);
  if (!workspace) return fail(GDR_ERR_INVALID, "gdr_chunk_fwd_train needs the backward workspace");
  if (workspace_bytes < L.total)
    return fail(GDR_ERR_INVALID, "workspace of %lld bytes given, %lld required", (long long)workspace_bytes,
                (long long)L.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(GDR_ERR_INVALID, "workspace must be 256-byte aligned");
  const hipError_t e = gdr::launch_chunk_train(*a, L, static_cast<unsigned char*>(workspace), stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "chunk forward (training) launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

int gdr_chunk_bwd_saved(const gdr_args* a, const gdr_grads* g, void* workspace, int64_t workspace_bytes,
                        hipStream_t stream) {
  const int rc = check_bwd(a, g, workspace, workspace_bytes);
  if (rc) return rc;
  const gdr::BwdLayout L = gdr::chunk_bwd_layout(*a);
  const hipError_t e = gdr::launch_chunk_bwd(*a, *g, L, static_cast<unsigned char*>(workspace), stream);
  if (e != hipSuccess) return fail(GDR_ERR_HIP, "chunk backward launch failed: %s", hipGetErrorString(e));
  g_last_error.clear();
  return GDR_OK;
}

}  // extern "C"
