// Torch binding of the C ABI for the Python entry points' common case: every
// argument a torch tensor with the expected dtype, shape and contiguity on the
// current GPU.  It validates in C++ (the per-call host cost of the reference's
// own pybind entry, kernel.cu:1066-1068, instead of ~15 us of Python checks)
// and calls gdn_decode_fwd / gdn_prefill_fwd on the stream it is given.
// Anything outside that case returns kNotFast without launching, and the
// Python entry then runs its full checks, which raise the descriptive errors.
#include <torch/extension.h>

#include <cmath>

#include "../../include/gdn_mi355x.h"

namespace {

constexpr int kNotFast = -100;

bool dense(const at::Tensor& t, at::ScalarType st, at::IntArrayRef shape, int64_t dev) {
  return t.defined() && t.scalar_type() == st && t.sizes().equals(shape) && t.is_contiguous() && t.is_cuda() &&
         t.get_device() == dev;
}

float resolve_scale(double scale) {
  return scale == 0.0 ? static_cast<float>(1.0 / std::sqrt(128.0)) : static_cast<float>(scale);
}

// launch_gdn(q, k, v, state, A_log, a, dt_bias, b, scale, out, new_state) of
// gdn_decode_qk4_v8_d128_k_last/solution/cuda/kernel.cu:982-1064, with out and
// new_state given; dev is the current device, stream its current stream.
int decode(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& state,
           const at::Tensor& A_log, const at::Tensor& a, const at::Tensor& dt_bias, const at::Tensor& b, double scale,
           const at::Tensor& out, const at::Tensor& new_state, int64_t rows_per_wave, int64_t stream, int64_t dev) {
  if (!q.defined() || q.dim() != 4) return kNotFast;
  const int64_t B = q.size(0);
  const auto bf = at::kBFloat16, f32 = at::kFloat;
  if (!dense(q, bf, {B, 1, 4, 128}, dev) || !dense(k, bf, {B, 1, 4, 128}, dev) ||
      !dense(v, bf, {B, 1, 8, 128}, dev) || !dense(state, f32, {B, 8, 128, 128}, dev) ||
      !dense(A_log, f32, {8}, dev) || !dense(dt_bias, f32, {8}, dev) || !dense(a, bf, {B, 1, 8}, dev) ||
      !dense(b, bf, {B, 1, 8}, dev) || !dense(new_state, f32, {B, 8, 128, 128}, dev))
    return kNotFast;
  if (!dense(out, bf, {B, 8, 128}, dev) && !dense(out, bf, {B, 1, 8, 128}, dev)) return kNotFast;
  if (B > 0 && state.data_ptr() == new_state.data_ptr()) return kNotFast;
  if (rows_per_wave != 0 && rows_per_wave != 16 && rows_per_wave != 32) return kNotFast;
  if (B == 0) return GDN_OK;
  if (B > 0x7fffffffLL) return kNotFast;
  return gdn_decode_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), state.data_ptr<float>(), A_log.data_ptr<float>(),
                        a.data_ptr(), dt_bias.data_ptr<float>(), b.data_ptr(), resolve_scale(scale), out.data_ptr(),
                        new_state.data_ptr<float>(), static_cast<int>(B), static_cast<int>(rows_per_wave),
                        reinterpret_cast<void*>(stream));
}

// launch_gdn(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
// new_state) of gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:56-262
// with output and new_state given; state may be None (zeros); without a
// workspace one of the default size comes from torch's caching allocator.
int prefill(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const c10::optional<at::Tensor>& state,
            const at::Tensor& A_log, const at::Tensor& a, const at::Tensor& dt_bias, const at::Tensor& b,
            const at::Tensor& cu_seqlens, double scale, const at::Tensor& output, const at::Tensor& new_state,
            const c10::optional<at::Tensor>& workspace, int64_t stream, int64_t dev) {
  if (!q.defined() || q.dim() != 3 || !cu_seqlens.defined() || cu_seqlens.dim() != 1 || cu_seqlens.numel() < 1)
    return kNotFast;
  const int64_t T = q.size(0), N = cu_seqlens.numel() - 1;
  const auto bf = at::kBFloat16, f32 = at::kFloat;
  const auto cut = cu_seqlens.scalar_type();
  if (cut != at::kInt && cut != at::kLong) return kNotFast;
  if (!dense(q, bf, {T, 4, 128}, dev) || !dense(k, bf, {T, 4, 128}, dev) || !dense(v, bf, {T, 8, 128}, dev) ||
      !dense(A_log, f32, {8}, dev) || !dense(dt_bias, f32, {8}, dev) || !dense(a, bf, {T, 8}, dev) ||
      !dense(b, bf, {T, 8}, dev) || !dense(cu_seqlens, cut, {N + 1}, dev) || !dense(output, bf, {T, 8, 128}, dev) ||
      !dense(new_state, f32, {N, 8, 128, 128}, dev))
    return kNotFast;
  const float* sp = nullptr;
  if (state.has_value() && state->defined()) {
    if (!dense(*state, f32, {N, 8, 128, 128}, dev)) return kNotFast;
    if (N > 0 && state->data_ptr() == new_state.data_ptr()) return kNotFast;
    sp = state->data_ptr<float>();
  }
  if (N == 0) return GDN_OK;
  if (N > 0x7fffffffLL) return kNotFast;
  at::Tensor ws;
  if (workspace.has_value() && workspace->defined()) {
    ws = *workspace;
    if (ws.scalar_type() != at::kByte || ws.dim() != 1 || !ws.is_contiguous() || !ws.is_cuda() ||
        ws.get_device() != dev ||
        static_cast<size_t>(ws.numel()) < gdn_prefill_workspace_min_bytes(static_cast<int>(N), T))
      return kNotFast;
  } else {
    ws = at::empty({static_cast<int64_t>(gdn_prefill_workspace_bytes(static_cast<int>(N), T))},
                   q.options().dtype(at::kByte));
  }
  return gdn_prefill_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), sp, A_log.data_ptr<float>(), a.data_ptr(),
                         dt_bias.data_ptr<float>(), b.data_ptr(), cu_seqlens.data_ptr(), cut == at::kLong ? 1 : 0,
                         static_cast<int>(N), T, resolve_scale(scale), output.data_ptr(), new_state.data_ptr<float>(),
                         ws.data_ptr(), static_cast<size_t>(ws.numel()), reinterpret_cast<void*>(stream));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.attr("NOT_FAST") = kNotFast;
  // the C ABI this binding was compiled against (gdn_mi355x.h); the loader
  // refuses the binding when the library reports another version
  m.attr("ABI") = GDN_ABI_VERSION;
  m.def("decode", &decode);
  m.def("prefill", &prefill);
}
