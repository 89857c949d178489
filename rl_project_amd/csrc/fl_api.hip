// C ABI of libflsampler.so: argument validation and kernel dispatch.
// Declarations and conventions: include/fl_sampler.h.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "fl_kernels.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return FL_OK;
}

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(FL_EIO, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

int validate_sample(const fl_sample_args* a, const char* fn) {
  if (a == nullptr) return fail(FL_EINVAL, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(fl_sample_args))
    return fail(FL_EINVAL, "%s: struct_size %u != %zu (header/library mismatch)", fn, a->struct_size,
                sizeof(fl_sample_args));
  if (a->dtype != FL_DTYPE_F32 && a->dtype != FL_DTYPE_BF16 && a->dtype != FL_DTYPE_F16)
    return fail(FL_EINVAL, "%s: unknown dtype %d", fn, a->dtype);
  if (a->batch < 0) return fail(FL_EINVAL, "%s: batch %lld < 0", fn, static_cast<long long>(a->batch));
  if (a->batch > 0x7fffffff) return fail(FL_ENOTSUP, "%s: batch %lld too large", fn, static_cast<long long>(a->batch));
  if (a->vocab < 1) return fail(FL_EINVAL, "%s: vocab %lld < 1", fn, static_cast<long long>(a->vocab));
  const int64_t vmax = a->dtype == FL_DTYPE_F32 ? FL_MAX_VOCAB_F32 : FL_MAX_VOCAB_16;
  if (a->vocab > vmax)
    return fail(FL_ENOTSUP, "%s: vocab %lld exceeds the library's limit %lld for dtype %d", fn,
                static_cast<long long>(a->vocab), static_cast<long long>(vmax), a->dtype);
  if (a->ld < a->vocab) return fail(FL_EINVAL, "%s: ld %lld < vocab %lld", fn, static_cast<long long>(a->ld),
                                    static_cast<long long>(a->vocab));
  if (a->batch > 0 && a->logits == nullptr) return fail(FL_EINVAL, "%s: logits is NULL", fn);
  if (!(a->softcap >= 0.0f) || std::isinf(a->softcap)) return fail(FL_EINVAL, "%s: softcap must be finite and >= 0", fn);
  if (a->hist_ids != nullptr && (a->hist_len == nullptr || a->hist_ld < 0))
    return fail(FL_EINVAL, "%s: hist_ids needs hist_len and hist_ld >= 0", fn);
  if (a->n_stop < 0 || (a->n_stop > 0 && (a->stop_ids == nullptr || a->stop_ld < 0)))
    return fail(FL_EINVAL, "%s: stop_ids/n_stop/stop_ld inconsistent", fn);
  if ((a->flags & ~(FL_FLAG_NO_SELECT | FL_FLAG_APPEND_HISTORY | FL_FLAG_EXACT_COUNTS | FL_FLAG_ONLY_LIMITED)) != 0)
    return fail(FL_EINVAL, "%s: unknown flags 0x%x", fn, static_cast<unsigned>(a->flags));
  if ((a->flags & FL_FLAG_ONLY_LIMITED) && (!(a->flags & FL_FLAG_EXACT_COUNTS) || a->out_status == nullptr))
    return fail(FL_EINVAL, "%s: FL_FLAG_ONLY_LIMITED needs FL_FLAG_EXACT_COUNTS and out_status", fn);
  if (a->uniform_div < 0) return fail(FL_EINVAL, "%s: uniform_div %lld < 0", fn, static_cast<long long>(a->uniform_div));
  if ((a->flags & FL_FLAG_APPEND_HISTORY) &&
      (a->hist_ids == nullptr || a->hist_ld <= 0 || (a->flags & FL_FLAG_NO_SELECT)))
    return fail(FL_EINVAL, "%s: FL_FLAG_APPEND_HISTORY needs per-row histories (hist_ld > 0) and a selection", fn);
  if (a->batch > 0 && (a->temperature == nullptr || a->top_k == nullptr || a->top_p == nullptr ||
                       a->min_p == nullptr || a->rep_penalty == nullptr))
    return fail(FL_EINVAL, "%s: the per-row parameter arrays (temperature, top_k, top_p, min_p, rep_penalty) "
                           "are required", fn);
  return FL_OK;
}

}  // namespace

extern "C" {

int fl_abi_version(void) { return FL_ABI_VERSION; }

const char* fl_last_error(void) { return g_error.c_str(); }

int fl_sample(const fl_sample_args* a, void* stream) {
  int rc = validate_sample(a, "fl_sample");
  if (rc != FL_OK) return rc;
  const bool select = (a->flags & FL_FLAG_NO_SELECT) == 0;
  if (select && a->out_token == nullptr) return fail(FL_EINVAL, "fl_sample: out_token is NULL");
  if (select && a->batch > 0 && a->uniforms == nullptr)
    return fail(FL_EINVAL, "fl_sample: uniforms is NULL (one draw per row is required unless FL_FLAG_NO_SELECT)");
  if (a->batch == 0) return ok();
  // (float32 rows have no 16-bit counters: a repeat for limited rows has nothing to do)
  if (a->dtype == FL_DTYPE_F32 && (a->flags & FL_FLAG_ONLY_LIMITED)) return ok();
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = a->dtype == FL_DTYPE_F32 ? fl::launch_sample_rows32(*a, s) : fl::launch_sample_rows16(*a, s);
  return check_launch(e, "fl_sample");
}

int fl_apply_filter(const fl_sample_args* a, const fl_row_desc* desc, void* out_filtered, int64_t out_ld,
                    float* out_probs, uint32_t* out_mask, void* stream) {
  int rc = validate_sample(a, "fl_apply_filter");
  if (rc != FL_OK) return rc;
  if (desc == nullptr) return fail(FL_EINVAL, "fl_apply_filter: desc is NULL");
  if (out_filtered != nullptr && out_ld < a->vocab) return fail(FL_EINVAL, "fl_apply_filter: out_ld < vocab");
  if (a->batch > 65535) return fail(FL_ENOTSUP, "fl_apply_filter: batch %lld exceeds 65535",
                                    static_cast<long long>(a->batch));
  if (a->batch == 0 || (out_filtered == nullptr && out_probs == nullptr && out_mask == nullptr)) return ok();
  const hipError_t e =
      fl::launch_apply_filter(*a, desc, out_filtered, out_ld, out_probs, out_mask, static_cast<hipStream_t>(stream));
  return check_launch(e, "fl_apply_filter");
}

// The checks shared by fl_spec_verify and fl_spec_verify_static; 1 = go on.
int validate_spec(const fl_spec_args* a, const char* fn) {
  if (a == nullptr) return fail(FL_EINVAL, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(fl_spec_args)) return fail(FL_EINVAL, "%s: struct_size mismatch", fn);
  if (a->dtype != FL_DTYPE_F32 && a->dtype != FL_DTYPE_BF16 && a->dtype != FL_DTYPE_F16)
    return fail(FL_EINVAL, "%s: unknown dtype %d", fn, a->dtype);
  if (a->batch < 0 || a->k < 1 || a->vocab < 1 || a->ld < a->vocab)
    return fail(FL_EINVAL, "%s: bad shape batch=%lld k=%lld vocab=%lld ld=%lld", fn,
                static_cast<long long>(a->batch), static_cast<long long>(a->k), static_cast<long long>(a->vocab),
                static_cast<long long>(a->ld));
  if (a->vocab > FL_MAX_VOCAB_F32 || a->batch > 0x7fffffff)
    return fail(FL_ENOTSUP, "%s: vocab %lld or batch %lld beyond the library's limits", fn,
                static_cast<long long>(a->vocab), static_cast<long long>(a->batch));
  if (a->batch == 0) return ok();
  if (!a->temperature || !a->target || !a->draft || !a->target_desc || !a->draft_desc || !a->draft_ids || !a->u_accept ||
      !a->u_resample || !a->bonus_token || !a->out_n_accepted || !a->out_tokens)
    return fail(FL_EINVAL, "%s: a required pointer is NULL", fn);
  return 1;
}

int fl_spec_verify(const fl_spec_args* a, void* stream) {
  const int v = validate_spec(a, "fl_spec_verify");
  if (v != 1) return v;
  if (a->workspace != nullptr && (a->workspace_bytes < 0 ||
                                  static_cast<size_t>(a->workspace_bytes) < fl::spec_workspace_bytes(a->batch)))
    return fail(FL_EINVAL, "fl_spec_verify: workspace of %lld bytes, %zu needed", static_cast<long long>(a->workspace_bytes),
                fl::spec_workspace_bytes(a->batch));
  if (a->workspace != nullptr && (reinterpret_cast<uintptr_t>(a->workspace) & 7u) != 0)
    return fail(FL_EINVAL, "fl_spec_verify: workspace not 8-byte aligned");
  const hipError_t e = fl::launch_spec_verify(*a, static_cast<hipStream_t>(stream));
  return check_launch(e, "fl_spec_verify");
}

int fl_spec_verify_static(const fl_spec_args* a, void* stream) {
  const int v = validate_spec(a, "fl_spec_verify_static");
  if (v != 1) return v;
  if (a->workspace != nullptr || a->workspace_bytes != 0)
    return fail(FL_EINVAL, "fl_spec_verify_static: workspace must be NULL with workspace_bytes 0 (the library's "
                "static scratch is used)");
  if (a->batch > FL_SPEC_STATIC_MAX_BATCH || fl::spec_workspace_bytes(a->batch) > fl::spec_static_scratch_bytes())
    return fail(FL_ENOTSUP, "fl_spec_verify_static: batch %lld exceeds the %d sequences of the static scratch",
                static_cast<long long>(a->batch), FL_SPEC_STATIC_MAX_BATCH);
  const hipError_t e = fl::launch_spec_verify_static(*a, static_cast<hipStream_t>(stream));
  return check_launch(e, "fl_spec_verify_static");
}

int fl_row_stats(const fl_row_stats_args* a, void* stream) {
  if (a == nullptr) return fail(FL_EINVAL, "fl_row_stats: args is NULL");
  if (a->struct_size != sizeof(fl_row_stats_args)) return fail(FL_EINVAL, "fl_row_stats: struct_size mismatch");
  if (a->dtype != FL_DTYPE_F32 && a->dtype != FL_DTYPE_BF16 && a->dtype != FL_DTYPE_F16)
    return fail(FL_EINVAL, "fl_row_stats: unknown dtype %d", a->dtype);
  if (a->rows < 0 || a->vocab < 1 || a->ld < a->vocab || (a->ref_logits && a->ref_ld < a->vocab))
    return fail(FL_EINVAL, "fl_row_stats: bad shape rows=%lld vocab=%lld ld=%lld ref_ld=%lld",
                static_cast<long long>(a->rows), static_cast<long long>(a->vocab), static_cast<long long>(a->ld),
                static_cast<long long>(a->ref_ld));
  if (a->vocab > FL_MAX_VOCAB_STATS || a->rows > 0x7fffffff)
    return fail(FL_ENOTSUP, "fl_row_stats: vocab %lld or rows %lld beyond the library's limits",
                static_cast<long long>(a->vocab), static_cast<long long>(a->rows));
  if (a->out_kl && !a->ref_logits) return fail(FL_EINVAL, "fl_row_stats: out_kl needs ref_logits");
  if (a->out_logprob && !a->labels) return fail(FL_EINVAL, "fl_row_stats: out_logprob needs labels");
  if (a->rows == 0) return ok();
  if (!a->logits) return fail(FL_EINVAL, "fl_row_stats: logits is NULL");
  const hipError_t e = fl::launch_row_stats(*a, static_cast<hipStream_t>(stream));
  return check_launch(e, "fl_row_stats");
}

int fl_lm_head_workspace_bytes(int64_t batch, int64_t vocab, size_t* out_bytes) {
  if (out_bytes == nullptr) return fail(FL_EINVAL, "fl_lm_head_workspace_bytes: out_bytes is NULL");
  if (batch < 0 || batch > FL_LM_HEAD_MAX_BATCH || vocab < 1 || vocab > FL_MAX_VOCAB_16)
    return fail(FL_EINVAL, "fl_lm_head_workspace_bytes: bad batch %lld or vocab %lld", static_cast<long long>(batch),
                static_cast<long long>(vocab));
  *out_bytes = fl::lm_head_workspace_bytes(batch, vocab);
  return ok();
}

int fl_lm_head_sample(const fl_lm_head_args* a, void* stream) {
  const char* fn = "fl_lm_head_sample";
  if (a == nullptr) return fail(FL_EINVAL, "%s: args is NULL", fn);
  if (a->struct_size != sizeof(fl_lm_head_args)) return fail(FL_EINVAL, "%s: struct_size mismatch", fn);
  if (a->dtype != FL_DTYPE_BF16) return fail(FL_ENOTSUP, "%s: dtype %d (bf16 only)", fn, a->dtype);
  if (a->batch < 0 || a->vocab < 1 || a->dim < 64 || a->dim % 64 != 0 || a->ld_hidden < a->dim)
    return fail(FL_EINVAL, "%s: bad shape batch=%lld dim=%lld vocab=%lld ld_hidden=%lld (dim a multiple of 64)", fn,
                static_cast<long long>(a->batch), static_cast<long long>(a->dim), static_cast<long long>(a->vocab),
                static_cast<long long>(a->ld_hidden));
  if (a->batch > FL_LM_HEAD_MAX_BATCH || a->vocab > FL_MAX_VOCAB_16 || a->dim > 16384 ||
      a->batch * a->ld_hidden > (1ll << 29))
    return fail(FL_ENOTSUP, "%s: batch %lld, vocab %lld or dim %lld beyond the library's limits (%d, %d, 16384)", fn,
                static_cast<long long>(a->batch), static_cast<long long>(a->vocab), static_cast<long long>(a->dim),
                FL_LM_HEAD_MAX_BATCH, FL_MAX_VOCAB_16);
  if (!std::isfinite(a->softcap) || a->softcap < 0.0f)
    return fail(FL_EINVAL, "%s: softcap must be finite and >= 0", fn);
  if (a->batch == 0) return ok();
  if (!a->hidden || !a->weight || !a->temperature || !a->top_k || !a->top_p || !a->min_p || !a->uniforms ||
      !a->out_token || !a->out_status)
    return fail(FL_EINVAL, "%s: a required pointer is NULL", fn);
  if (a->hist_ids != nullptr && (a->hist_len == nullptr || a->hist_ld < 0))
    return fail(FL_EINVAL, "%s: hist_ids needs hist_len and hist_ld >= 0", fn);
  if (a->workspace == nullptr || a->workspace_bytes < 0 ||
      static_cast<size_t>(a->workspace_bytes) < fl::lm_head_workspace_bytes(a->batch, a->vocab))
    return fail(FL_EINVAL, "%s: workspace of %lld bytes, %zu needed", fn, static_cast<long long>(a->workspace_bytes),
                fl::lm_head_workspace_bytes(a->batch, a->vocab));
  if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0)
    return fail(FL_EINVAL, "%s: workspace not 256-byte aligned", fn);
  if ((reinterpret_cast<uintptr_t>(a->hidden) & 15u) != 0 || (reinterpret_cast<uintptr_t>(a->weight) & 15u) != 0 ||
      (a->ld_hidden % 8) != 0)
    return fail(FL_EINVAL, "%s: hidden and weight must be 16-byte aligned (ld_hidden a multiple of 8)", fn);
  const hipError_t e = fl::launch_lm_head(*a, static_cast<hipStream_t>(stream));
  return check_launch(e, fn);
}

int fl_spec_workspace_bytes(int64_t batch, size_t* out_bytes) {
  if (out_bytes == nullptr) return fail(FL_EINVAL, "fl_spec_workspace_bytes: out_bytes is NULL");
  if (batch < 0 || batch > 0x7fffffff)
    return fail(FL_EINVAL, "fl_spec_workspace_bytes: bad batch %lld", static_cast<long long>(batch));
  *out_bytes = fl::spec_workspace_bytes(batch);
  return ok();
}

int fl_spec_cache_workspace_bytes(int64_t batch, int64_t vocab, size_t* out_bytes) {
  if (out_bytes == nullptr) return fail(FL_EINVAL, "fl_spec_cache_workspace_bytes: out_bytes is NULL");
  if (batch < 0 || batch > 0x7fffffff || vocab < 1 || vocab > FL_MAX_VOCAB_F32)
    return fail(FL_EINVAL, "fl_spec_cache_workspace_bytes: bad batch %lld or vocab %lld", static_cast<long long>(batch),
                static_cast<long long>(vocab));
  *out_bytes = fl::spec_cache_workspace_bytes(batch, vocab);
  return ok();
}

}  // extern "C"
