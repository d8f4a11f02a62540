// GDN decode: one token per sequence, one HBM-streaming pass over the state.
//
// Per (batch n, v-head h), state S = state[n, h] is [V=128, K=128] fp32 (k-last):
//   g     = exp(-exp(A_log[h]) * softplus(a[n,h] + dt_bias[h])),  beta = sigmoid(b[n,h])
//   p     = g (S k)            r = g (S q)            (row dots over K)
//   delta = beta (v - p)
//   S'    = g S + delta k^T
//   o     = scale S' q = scale (r + delta (k . q))
// Semantics follow gdn_decode_qk4_v8_d128_k_last/solution/reference_torch_impl.py:36-69;
// the entry point replaces launch_gdn in solution/cuda/kernel.cu:982-1064.
//
// Mapping (wave64): a workgroup is one wave and owns ROWS consecutive v-rows of
// one (n, h) tile.  Lane l = 32*half + lam reads columns [4 lam, 4 lam + 4) of
// rows v0 + half*ROWS/2 + i, i < ROWS/2, with one 16-byte load per row, so every
// load instruction of the wave covers two whole 512-byte rows.  Each state byte
// is read once and written once (non-temporal loads and stores).  The 2*ROWS/2 row dots
// (S k and S q for each row) are reduced over the 32 lanes of each half with a
// reduce-scatter butterfly (DPP / ds_swizzle), which leaves exactly one fully
// reduced value per lane; delta is then broadcast to the half through LDS.
#include "gdn_common.h"
#include "../../include/gdn_mi355x.h"

namespace gdn {

template <int MASK, int N>
__device__ __forceinline__ void reduce_scatter_step(float* v, bool upper) {
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    const float send = upper ? v[j] : v[j + N / 2];
    const float keep = upper ? v[j + N / 2] : v[j];
    v[j] = keep + xor_lane<MASK>(send);
  }
}

// ROWS rows of one head per wave (ROWS/2 per half-wave).
template <int ROWS>
__global__ __launch_bounds__(64) void decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ state,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b, float scale,
    uint16_t* __restrict__ out, float* __restrict__ new_state) {
  constexpr int NL = ROWS / 2;            // rows per half-wave == loads per lane
  constexpr int NV = 2 * NL;              // values reduced per half-wave
  static_assert(NV == 16 || NV == 32, "ROWS must be 8 or 16 per half-wave");
  constexpr int kTiles = kDim / ROWS;

  __shared__ float delta_lds[2][NL];

  const int lane = threadIdx.x;
  const int half = lane >> 5;
  const int lam = lane & 31;
  const int nh = blockIdx.x / kTiles;     // n * 8 + h
  const int vt = blockIdx.x - nh * kTiles;
  const int h = nh & (kVHeads - 1);
  const int n = nh >> 3;
  const int hq = h / kGva;
  const int row0 = vt * ROWS + half * NL;

  // ---- issue the state loads first (the only large traffic) ----
  // Non-temporal: every state byte is read exactly once, so the loads stream
  // instead of allocating in L2 / MALL (measured on MI355X at B = 64: 11.84 ->
  // 10.84 us per step with plain vs non-temporal loads, same outputs).
  const float* src = state + static_cast<size_t>(nh) * kHeadState + row0 * kDim + lam * 4;
  f32x4 s[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) s[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + i * kDim));

  // ---- q, k for this lane's 4 columns; gates for this (n, h) ----
  const size_t qk_off = (static_cast<size_t>(n) * kQKHeads + hq) * kDim + lam * 4;
  const uint2 kraw = *reinterpret_cast<const uint2*>(k + qk_off);
  const uint2 qraw = *reinterpret_cast<const uint2*>(q + qk_off);
  const float kc[4] = {bf_lo(kraw.x), bf_hi(kraw.x), bf_lo(kraw.y), bf_hi(kraw.y)};
  const float qc[4] = {bf_lo(qraw.x), bf_hi(qraw.x), bf_lo(qraw.y), bf_hi(qraw.y)};
  const float g = expf(log_decay(A_log[h], bf2f(a[nh]), dt_bias[h]));
  const float beta = sigmoidf(bf2f(b[nh]));
  float kq = kc[0] * qc[0] + kc[1] * qc[1] + kc[2] * qc[2] + kc[3] * qc[3];
  kq = half_wave_allreduce(kq);

  // ---- partial row dots: vals[i] = S_i . k, vals[NL + i] = S_i . q ----
  float vals[NV];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    vals[i] = s[i].x * kc[0] + s[i].y * kc[1] + s[i].z * kc[2] + s[i].w * kc[3];
    vals[NL + i] = s[i].x * qc[0] + s[i].y * qc[1] + s[i].z * qc[2] + s[i].w * qc[3];
  }
  // reduce-scatter over the 32 lanes of the half: afterwards lane lam holds the
  // full sum of value index lam >> (5 - log2 NV)
  reduce_scatter_step<16, NV>(vals, lam & 16);
  reduce_scatter_step<8, NV / 2>(vals, lam & 8);
  reduce_scatter_step<4, NV / 4>(vals, lam & 4);
  reduce_scatter_step<2, NV / 8>(vals, lam & 2);
  float red;
  if constexpr (NV == 32) {
    reduce_scatter_step<1, 2>(vals, lam & 1);
    red = vals[0];
  } else {
    red = xor_sum<1>(vals[0]);
  }
  constexpr int kShift = (NV == 32) ? 0 : 1;
  const int idx = lam >> kShift;          // value index held by this lane
  const int row_i = idx & (NL - 1);       // row within the half
  const bool is_q = idx >= NL;

  // p-lanes: delta_i = beta (v_i - g p_i); q-lanes fetch it from lane lam ^ 16
  const float vrow = bf2f(v[static_cast<size_t>(nh) * kDim + row0 + row_i]);
  const float delta = beta * (vrow - g * red);
  const float delta_x = xor_lane<16>(delta);
  if (!is_q && ((lam & kShift) == 0)) delta_lds[half][row_i] = delta;
  if (is_q && ((lam & kShift) == 0)) {
    const float o = scale * (g * red + delta_x * kq);
    out[static_cast<size_t>(nh) * kDim + row0 + row_i] = f2bf(o);
  }
  __syncthreads();

  // ---- S' = g S + delta k^T, streamed back once ----
  float* dst = new_state + static_cast<size_t>(nh) * kHeadState + row0 * kDim + lam * 4;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const float d = delta_lds[half][i];
    f32x4 r;
    r.x = fmaf(d, kc[0], g * s[i].x);
    r.y = fmaf(d, kc[1], g * s[i].y);
    r.z = fmaf(d, kc[2], g * s[i].z);
    r.w = fmaf(d, kc[3], g * s[i].w);
    __builtin_nontemporal_store(r, reinterpret_cast<f32x4*>(dst + i * kDim));
  }
}

}  // namespace gdn

extern "C" int gdn_decode_fwd(const void* q, const void* k, const void* v, const float* state,
                              const float* A_log, const void* a, const float* dt_bias,
                              const void* b, float scale, void* out, float* new_state,
                              int batch, int rows_per_wave, void* stream) {
  using namespace gdn;
  if (batch < 0) return GDN_ERR_INVALID_ARGUMENT;
  if (batch == 0) return GDN_OK;
  if (!q || !k || !v || !state || !A_log || !a || !dt_bias || !b || !out || !new_state)
    return GDN_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(state) | reinterpret_cast<uintptr_t>(new_state)) & 15u)
    return GDN_ERR_UNALIGNED;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) & 7u)
    return GDN_ERR_UNALIGNED;
  // v, a, b, out: 2-byte accesses; A_log, dt_bias: 4-byte
  if ((reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
       reinterpret_cast<uintptr_t>(out)) & 1u)
    return GDN_ERR_UNALIGNED;
  if ((reinterpret_cast<uintptr_t>(A_log) | reinterpret_cast<uintptr_t>(dt_bias)) & 3u) return GDN_ERR_UNALIGNED;
  if (state == new_state) return GDN_ERR_ALIASING;
  if (!(scale > 0.0f) && !(scale < 0.0f)) scale = 0.08838834764831845f;  // 0 / NaN -> 1/sqrt(128)
  if (rows_per_wave == 0) rows_per_wave = (batch >= 16) ? 32 : 16;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  const auto* ab = static_cast<const uint16_t*>(a);
  const auto* bb = static_cast<const uint16_t*>(b);
  auto* ob = static_cast<uint16_t*>(out);
  const long heads = static_cast<long>(batch) * kVHeads;
  if (rows_per_wave == 32) {
    const long grid = heads * (kDim / 32);
    if (grid > 0x7fffffffL) return GDN_ERR_INVALID_ARGUMENT;
    decode_kernel<32><<<dim3(static_cast<unsigned>(grid)), dim3(64), 0, st>>>(
        qb, kb, vb, state, A_log, ab, dt_bias, bb, scale, ob, new_state);
  } else if (rows_per_wave == 16) {
    const long grid = heads * (kDim / 16);
    if (grid > 0x7fffffffL) return GDN_ERR_INVALID_ARGUMENT;
    decode_kernel<16><<<dim3(static_cast<unsigned>(grid)), dim3(64), 0, st>>>(
        qb, kb, vb, state, A_log, ab, dt_bias, bb, scale, ob, new_state);
  } else {
    return GDN_ERR_INVALID_ARGUMENT;
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? GDN_OK : static_cast<int>(err);
}
