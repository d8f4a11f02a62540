// GDN prefill: chunked (C = 64) y-space WY recurrence on gfx950 bf16 MFMA.
//
// For one v-head and one chunk of c <= 64 tokens with incoming state S ([V, K]),
// let Gam_t = sum_{i<=t} log g_i (within the chunk), rho[t,i] = exp(Gam_t - Gam_i):
//   A     = I + strict_lower(beta_t rho[t,i] k_t.k_i),   Tb = A^{-1} diag(beta)
//   Aqk   = lower(rho[t,i] q_t.k_i)
//   Delta = Tb (V - diag(gam) K S^T)                     gam_t = exp(Gam_t)
//   O     = scale (diag(gam) Q S^T + Aqk Delta)
//   S'    = gam_c S + (diag(tail) Delta)^T K             tail_t = exp(Gam_c - Gam_t)
// which equals the token recurrence of
// gdn_prefill_qk4_v8_d128_k_last/solution/reference_torch_impl.py:66-88 exactly
// in real arithmetic.  All gate factors are bounded ratios (no division by a
// cumulative decay), so C = 64 is safe where the reference's X-space form
// (solution/triton/kernel.py:421-425) divides by G.
//
// Three launches, all on the caller's stream:
//   plan     : 1 work-group; chunk records (seq, first token, length) for all
//              sequences from cu_seqlens, with no host synchronisation.
//   prepass  : one work-group per (record, v-head), all records in parallel:
//              gates, K K^T / Q K^T on MFMA, fp32 blocked triangular inverse,
//              and the packed MFMA operands Tb (bf16 hi+lo), Aqk (bf16) plus
//              gam / tail, written to the workspace.
//   consumer : one work-group per (seq, v-head); each of its 8 waves (two per
//              SIMD) owns one 16-wide V tile and runs the whole chunk
//              recurrence for it with the state in MFMA registers; the chunk
//              operands (K, Q, V rows, packed Tb / Aqk, gates) are copied from
//              global memory straight into double-buffered LDS and shared by
//              the 8 waves.
//
// Precision policy (fp32 accumulation everywhere): K, Q, V are bf16 inputs, so
// their products are exact.  S enters K S^T and Q S^T as a single bf16; Tb and
// R = V - gam K S^T enter Delta = Tb R as bf16 hi+lo pairs (three MFMAs); the
// state update uses Delta' = tail Delta as a hi+lo pair; Aqk Delta (output only)
// is single bf16.  The fp32 state never leaves registers between chunks.
#include "gdn_common.h"
#include "../../include/gdn_mi355x.h"

namespace gdn {

constexpr int kChunk = 64;
constexpr int kFragElems = 4096;             // 64x64 bf16 operand in fragment order

// MFMA operands in "permuted fragment order".  For v_mfma_f32_16x16x32_bf16
// the hardware pairs slot s of lane group lg in A with the same slot of the
// same lane group in B, so the depth index behind each (lg, s) is ours to
// choose as long as A and B agree.  This build uses
//     depth(d, lg, s) = 32 d + 16 (s >> 2) + 4 lg + (s & 3)
// which is exactly the row index a 16x16 MFMA result (C layout: lane (lg, l16)
// holds rows 4 lg + rr of tiles 2d and 2d+1) already holds in its registers.
// Results of one MFMA can therefore be fed back as the B operand of the next
// with no cross-lane movement.  A 64x64 matrix M is stored as fragments
// (m = row tile, d = depth chunk): element ((m*2 + d)*64 + lane)*8 + s is
// M[16m + lane%16][depth(d, lane/16, s)].
__host__ __device__ constexpr int perm_depth(int d, int lg, int s) {
  return 32 * d + 16 * (s >> 2) + 4 * lg + (s & 3);
}

// ---- workspace layout -------------------------------------------------------
struct WsLayout {
  size_t frag_off;     // bf16 [R][8][3][4096]   (Tb hi, Tb lo, Aqk)
  size_t gam_off;      // f32  [R][8][2][64]     (gam, tail)
  size_t start_off;    // i32  [N + 1]           record start per sequence
  size_t rec_off;      // i32x4[R]               (seq, first token, length, 0)
  size_t total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline long long max_records(int num_seqs, long long tokens) {
  return (tokens + kChunk - 1) / kChunk + num_seqs;
}

__host__ __device__ inline WsLayout ws_layout(int num_seqs, long long tokens) {
  WsLayout L;
  const size_t R = static_cast<size_t>(max_records(num_seqs, tokens));
  size_t off = 0;
  L.frag_off = off;  off = align256(off + R * kVHeads * 3 * kFragElems * sizeof(uint16_t));
  L.gam_off = off;   off = align256(off + R * kVHeads * 2 * kChunk * sizeof(float));
  L.start_off = off; off = align256(off + (static_cast<size_t>(num_seqs) + 1) * sizeof(int));
  L.rec_off = off;   off = align256(off + R * sizeof(int4));
  L.total = off;
  return L;
}

// Sequence bounds from cu_seqlens, clamped into [0, T] with end >= start.
__device__ __forceinline__ void seq_bounds(const void* cu, int is64, int s, long long T,
                                           long long& t0, long long& t1) {
  long long a, b;
  if (is64) {
    a = static_cast<const long long*>(cu)[s];
    b = static_cast<const long long*>(cu)[s + 1];
  } else {
    a = static_cast<const int*>(cu)[s];
    b = static_cast<const int*>(cu)[s + 1];
  }
  a = a < 0 ? 0 : (a > T ? T : a);
  b = b < a ? a : (b > T ? T : b);
  t0 = a;
  t1 = b;
}

// ============================================================================
// plan: record numbering (exclusive scan of per-sequence chunk counts)
// ============================================================================
constexpr int kPlanThreads = 1024;

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(
    const void* __restrict__ cu, int is64, int num_seqs, long long T, int R,
    int* __restrict__ rec_start, int4* __restrict__ recs) {
  __shared__ int part[kPlanThreads];
  const int tid = threadIdx.x;
  const int per = (num_seqs + kPlanThreads - 1) / kPlanThreads;
  const int s_begin = tid * per;
  const int s_end = min(num_seqs, s_begin + per);
  int local = 0;
  for (int s = s_begin; s < s_end; ++s) {
    long long t0, t1;
    seq_bounds(cu, is64, s, T, t0, t1);
    local += static_cast<int>((t1 - t0 + kChunk - 1) / kChunk);
  }
  part[tid] = local;
  __syncthreads();
  // Hillis-Steele inclusive scan over the per-thread totals
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int add = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int base = part[tid] - local;
  const int total = min(part[kPlanThreads - 1], R);
  for (int s = s_begin; s < s_end; ++s) {
    long long t0, t1;
    seq_bounds(cu, is64, s, T, t0, t1);
    rec_start[s] = base;
    // overlapping (non-monotonic) cu_seqlens can ask for more than R records:
    // records past the capacity are dropped and the consumer skips them
    for (long long c0 = t0; c0 < t1; c0 += kChunk, ++base) {
      const int len = static_cast<int>(min(static_cast<long long>(kChunk), t1 - c0));
      if (base < R) recs[base] = make_int4(s, static_cast<int>(c0), len, 0);
    }
  }
  if (tid == 0) rec_start[num_seqs] = total;
  for (int r = total + tid; r < R; r += kPlanThreads) recs[r] = make_int4(-1, 0, 0, 0);
}

// ============================================================================
// device helpers shared by the prepass and the consumer
// ============================================================================
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// K / Q rows in LDS keep natural column order; the 16-byte chunk j of row t is
// stored at position j ^ kq_swz(t).  kq_swz is a bijection of t & 15, so the
// row reads (8 consecutive k of 16 rows) and the transposed reads (4
// consecutive k of 4 rows x 4 chunks) are bank-conflict free.
__device__ __forceinline__ int kq_swz(int t) { return ((t & 3) << 2) | ((t >> 2) & 3); }

// 16 bytes per lane from global memory straight into LDS: lane i of the wave
// writes bytes [16 i, 16 i + 16) after the wave-uniform LDS address.
__device__ __forceinline__ void dma16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, 0);
}

// ============================================================================
// prepass: chunk-local WY terms for one (record, v-head)
// ============================================================================
constexpr int kPrepassThreads = 256;
constexpr int kMRow = 68;     // floats per LDS row of the 64x64 fp32 matrices (16-byte aligned)

// 50 KB: three work-groups per CU.  T reuses the K / Q rows' space once the
// grams have been formed.
struct __align__(16) PrepassSmem {
  union {
    uint16_t kq[2][kChunk][kDim];   // K, Q rows (bf16, chunk-swizzled)
    float tm[kChunk][kMRow];        // T = (I + N)^{-1}
  } u;
  float nm[kChunk][kMRow];          // N = strict lower beta_t rho K K^T; upper blocks are scratch
  float lgam[kChunk];               // Gam_t / ln 2 (log2 cumulative decay)
  float beta[kChunk];
};

// j-th lower 16x16 tile (mi >= ni) of a 4x4 tile grid, row by row:
// (0,0) (1,0) (1,1) (2,0) (2,1) (2,2) (3,0) (3,1) (3,2) (3,3).
__device__ __forceinline__ void lower_tile(int j, int& mi, int& ni) {
  mi = j >= 6 ? 3 : (j >= 3 ? 2 : (j >= 1 ? 1 : 0));
  ni = j - mi * (mi + 1) / 2;
}

// acc += X Y for 16x16 fp32 blocks in LDS (row stride kMRow) on fp32 MFMA;
// result in C layout (lane (lg, l16) holds rows 4 lg .. 4 lg + 3 of column l16).
__device__ __forceinline__ f32x4 block_prod(f32x4 acc, const float* X, const float* Y, int l16, int lg) {
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
    acc = mfma_f32(X[l16 * kMRow + 4 * kc + lg], Y[(4 * kc + lg) * kMRow + l16], acc);
  return acc;
}

__device__ __forceinline__ void block_store(float* Z, const f32x4& v, float sc, int l16, int lg) {
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) Z[(4 * lg + rr) * kMRow + l16] = sc * v[rr];
}

__global__ __launch_bounds__(kPrepassThreads) void prepass_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const int4* __restrict__ recs, uint16_t* __restrict__ ws_frag,
    float* __restrict__ ws_gam) {
  __shared__ PrepassSmem sm;
  // linear id = r * 8 + h: v-head h runs on XCD h, as its consumer does
  const int r = blockIdx.x / kVHeads;
  const int h = blockIdx.x % kVHeads;
  const int hq = h / kGva;
  const int4 rec = recs[r];
  const int c = rec.z;
  if (c <= 0) return;
  const long long t0 = rec.y;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int lg = lane >> 4;

  // gate inputs first (wave 0, lane = token): their latency overlaps the row copies
  float a_t = 0.0f, b_t = 0.0f, alog = 0.0f, dtb = 0.0f;
  if (w == 0) {
    const size_t gi = (t0 + min(lane, c - 1)) * kVHeads + h;
    a_t = bf2f(a[gi]);
    b_t = bf2f(b[gi]);
    alog = A_log[h];
    dtb = dt_bias[h];
  }

  // ---- K, Q rows of the chunk, copied straight into LDS ----
  // Rows past the chunk end repeat row c-1: they meet beta = 0 (rows of N),
  // i <= t masks (columns) and rows of Aqk whose outputs are never stored.
  {
    const size_t qk0 = (static_cast<size_t>(t0) * kQKHeads + hq) * kDim;
    const char* kb = reinterpret_cast<const char*>(k + qk0);
    const char* qb = reinterpret_cast<const char*>(q + qk0);
    const int row0 = 4 * w + (lane >> 4);          // + 16 j keeps row & 15
    const uint32_t col = 16u * static_cast<uint32_t>((lane & 15) ^ kq_swz(row0));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t off = static_cast<uint32_t>(min(row0 + 16 * j, c - 1)) * (kQKHeads * kDim * 2) + col;
      dma16(kb + off, &sm.u.kq[0][16 * j + 4 * w][0]);
      dma16(qb + off, &sm.u.kq[1][16 * j + 4 * w][0]);
    }
  }

  // ---- gates (wave 0, lane = token): Gam_t inclusive scan of log2 g, beta ----
  if (w == 0) {
    const int t = lane;
    // clamp: g = e^-100 is already 0 to fp32 working precision, and a finite
    // floor keeps Gam finite (no -inf - -inf) for absurd gate inputs
    const float lgv = t < c ? fmaxf(log_decay(alog, a_t, dtb), -100.0f) * kLog2e : 0.0f;
    const float bet = t < c ? sigmoidf(b_t) : 0.0f;
    float scan = lgv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(scan, off, 64);
      if (lane >= off) scan += o;
    }
    sm.lgam[t] = scan;
    sm.beta[t] = bet;
    const float last = __shfl(scan, c - 1, 64);
    float* gp = ws_gam + (static_cast<size_t>(r) * kVHeads + h) * 2 * kChunk;
    gp[t] = t < c ? fast_exp2(scan) : 0.0f;
    gp[kChunk + t] = t < c ? fast_exp2(last - scan) : 0.0f;
  }
  __syncthreads();

  // ---- grams on MFMA: N (K K^T, to LDS) and Aqk (Q K^T, to the workspace) ----
  // Q K^T is formed transposed (A = K rows, B = Q rows): lane (lg, l16) then
  // holds Aqk[16 mi + l16][16 ni + 4 lg + rr], which is exactly half (slots
  // 4 (ni & 1) .. +3) of fragment (mi, ni >> 1) in permuted fragment order.
  uint16_t* frag = ws_frag + (static_cast<size_t>(r) * kVHeads + h) * 3 * kFragElems;
  const int rsw = kq_swz(l16);
  // wave w forms lower tiles j = w, w + 4, w + 8 (< 10) of both grams; all
  // twelve accumulator chains are independent, so their MFMAs interleave
  f32x4 akk[3], aqk[3];
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    int mi, ni;
    lower_tile(min(w + 4 * n, 9), mi, ni);
    akk[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    aqk[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int at = 8 * ((4 * d + lg) ^ rsw);
      const bf16x8 km = *reinterpret_cast<const bf16x8*>(&sm.u.kq[0][16 * mi + l16][at]);
      const bf16x8 kn = *reinterpret_cast<const bf16x8*>(&sm.u.kq[0][16 * ni + l16][at]);
      const bf16x8 qm = *reinterpret_cast<const bf16x8*>(&sm.u.kq[1][16 * mi + l16][at]);
      akk[n] = mfma16(km, kn, akk[n]);
      aqk[n] = mfma16(kn, qm, aqk[n]);
    }
  }
#pragma unroll
  for (int n = 0; n < 3; ++n) {
    if (w + 4 * n >= 10) break;   // wave-uniform
    int mi, ni;
    lower_tile(w + 4 * n, mi, ni);
    {
      // akk[n][rr] = K_t . K_i, t = 16 mi + 4 lg + rr, i = 16 ni + l16
      const int i = 16 * ni + l16;
      const float gi_ = sm.lgam[i];
      const f32x4 gt = *reinterpret_cast<const f32x4*>(&sm.lgam[16 * mi + 4 * lg]);
      const f32x4 bt = *reinterpret_cast<const f32x4*>(&sm.beta[16 * mi + 4 * lg]);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int t = 16 * mi + 4 * lg + rr;
        sm.nm[t][i] = i < t ? bt[rr] * fast_exp2(gt[rr] - gi_) * akk[n][rr] : 0.0f;
      }
    }
    {
      // aqk[n][rr] = K_i . Q_t (transposed), i = 16 ni + 4 lg + rr, t = 16 mi + l16
      const int t = 16 * mi + l16;
      const float gt = sm.lgam[t];
      const f32x4 gi4 = *reinterpret_cast<const f32x4*>(&sm.lgam[16 * ni + 4 * lg]);
      float x[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = 16 * ni + 4 * lg + rr;
        x[rr] = i <= t ? fast_exp2(gt - gi4[rr]) * aqk[n][rr] : 0.0f;
      }
      *reinterpret_cast<u32x2*>(frag + 2 * kFragElems + ((mi * 2 + (ni >> 1)) * 64 + lane) * 8 + 4 * (ni & 1)) =
          u32x2{pack_bf2(x[0], x[1]), pack_bf2(x[2], x[3])};
    }
  }
  // the six half-fragments of Aqk above the diagonal: (mi, ni) = (0,1) (0,2)
  // (0,3) (1,2) (1,3) (2,3)
  for (int z = tid; z < 6 * 64; z += kPrepassThreads) {
    const int zj = z >> 6, zl = z & 63;
    const int mi = zj < 3 ? 0 : (zj < 5 ? 1 : 2);
    const int ni = zj < 3 ? zj + 1 : (zj < 5 ? zj - 1 : 3);
    *reinterpret_cast<u32x2*>(frag + 2 * kFragElems + ((mi * 2 + (ni >> 1)) * 64 + zl) * 8 + 4 * (ni & 1)) =
        u32x2{0u, 0u};
  }
  __syncthreads();   // N complete; K / Q space becomes T

  // ---- T = (I + N)^{-1}: diagonal 16x16 blocks by forward substitution ----
  if (lane < 16) {
    const int base = 16 * w;
    const int j = lane;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = (i == j) ? 1.0f : 0.0f;
#pragma unroll
      for (int m2 = 0; m2 < i; ++m2) acc = fmaf(-sm.nm[base + i][base + m2], x[m2], acc);
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sm.u.tm[base + i][base + j] = x[i];
  }

  // ---- off-diagonal blocks by distance on fp32 MFMA:
  //      T_ij = -T_ii P,  P = sum_{m=j}^{i-1} N_im T_mj  (P staged in N's unused upper block (j, i))
#pragma unroll
  for (int dist = 1; dist < 4; ++dist) {
    __syncthreads();
    if (w < 4 - dist) {
      const int bj = w, bi = w + dist;
      f32x4 p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < dist; ++u)
        p = block_prod(p, &sm.nm[16 * bi][16 * (bj + u)], &sm.u.tm[16 * (bj + u)][16 * bj], l16, lg);
      float* scr = &sm.nm[16 * bj][16 * bi];
      block_store(scr, p, 1.0f, l16, lg);
      f32x4 tv = {0.f, 0.f, 0.f, 0.f};
      tv = block_prod(tv, &sm.u.tm[16 * bi][16 * bi], scr, l16, lg);
      block_store(&sm.u.tm[16 * bi][16 * bj], tv, -1.0f, l16, lg);
    }
  }
  __syncthreads();

  // ---- pack Tb = T diag(beta) as bf16 hi + lo (permuted fragment order) ----
  // fragment (m, d), lane l: row t = 16 m + l % 16, slots s: i = perm_depth(d, l / 16, s)
  for (int qi = tid; qi < 512; qi += kPrepassThreads) {
    const int m = qi >> 7, d = (qi >> 6) & 1, l = qi & 63;
    const int t = 16 * m + (l & 15);
    const int i0 = 32 * d + 4 * (l >> 4);
    const f32x4 ta = *reinterpret_cast<const f32x4*>(&sm.u.tm[t][i0]);
    const f32x4 tb = *reinterpret_cast<const f32x4*>(&sm.u.tm[t][i0 + 16]);
    const f32x4 ba = *reinterpret_cast<const f32x4*>(&sm.beta[i0]);
    const f32x4 bb = *reinterpret_cast<const f32x4*>(&sm.beta[i0 + 16]);
    float x[8];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      x[s] = i0 + s <= t ? ta[s] * ba[s] : 0.0f;
      x[4 + s] = i0 + 16 + s <= t ? tb[s] * bb[s] : 0.0f;
    }
    u32x4 wh, wl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wh[j] = pack_bf2(x[2 * j], x[2 * j + 1]);
      wl[j] = pack_bf2(x[2 * j] - bf_lo(wh[j]), x[2 * j + 1] - bf_hi(wh[j]));
    }
    *reinterpret_cast<u32x4*>(frag + qi * 8) = wh;
    *reinterpret_cast<u32x4*>(frag + kFragElems + qi * 8) = wl;
  }
}

// ============================================================================
// consumer: one work-group per (seq, v-head); wave w owns value rows 16w..16w+15
// ============================================================================
constexpr int kConsumerWaves = kDim / 16;  // 8: two waves per SIMD
constexpr int kConsumerThreads = 64 * kConsumerWaves;

// Chunk operands in LDS, double-buffered.  The buffer index is the outer index
// of every field (not of a struct of fields) so that buffer 1 of a field sits
// within a ds_read immediate offset of buffer 0.
//   ks / qs : K / Q rows in natural column order; the 16-byte chunk j of row t
//             is stored at position j ^ kq_swz(t), which makes the row reads
//             (8 consecutive k) and the transposed reads (4 consecutive k of 4
//             rows) bank-conflict free.
//   vs      : V rows; chunk j of row t at j ^ v_swz(t).
//   frag    : Tb hi, Tb lo, Aqk in permuted fragment order (lane-contiguous).
//   gt      : gam[64], tail[64] and 128 floats of padding.
// Rows t >= c of a partial chunk hold copies of row c-1 (finite data); they
// only meet zero rows / columns of Tb and Aqk and zero gam / tail.
struct __align__(16) ConsumerSmem {
  uint16_t ks[2][kChunk][kDim];
  uint16_t qs[2][kChunk][kDim];
  uint16_t vs[2][kChunk][kDim];
  uint16_t frag[2][3][kFragElems];
  float gt[2][4 * kChunk];
};

__device__ __forceinline__ int v_swz(int t) { return (t & 3) << 2; }

typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// gfx950 transposed LDS read: in each 16-lane group, lane i receives element
// (i & 3) of the 8-byte vectors addressed by lanes i/4, i/4+4, i/4+8, i/4+12.
__device__ __forceinline__ u32x2 lds_tr16(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ bf16x8 join_frag(u32x2 lo, u32x2 hi) {
  return __builtin_bit_cast(bf16x8, u32x4{lo.x, lo.y, hi.x, hi.y});
}


// Eight fp32 values in slot order -> bf16 fragment (hi) and the residual (lo).
__device__ __forceinline__ void split_frag(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = pack_bf2(x[2 * j], x[2 * j + 1]);
    l[j] = pack_bf2(x[2 * j] - bf_lo(h[j]), x[2 * j + 1] - bf_hi(h[j]));
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

__device__ __forceinline__ bf16x8 round_frag(const float (&x)[8]) {
  return __builtin_bit_cast(bf16x8, u32x4{pack_bf2(x[0], x[1]), pack_bf2(x[2], x[3]),
                                          pack_bf2(x[4], x[5]), pack_bf2(x[6], x[7])});
}

// The 8 slot values of permuted depth chunk d from four C-layout tiles
// (tile 2d + s/4, row 4 lg + s%4).
__device__ __forceinline__ void gather_slots(const f32x4 (&t)[4], int d, float (&x)[8]) {
#pragma unroll
  for (int s = 0; s < 8; ++s) x[s] = t[2 * d + (s >> 2)][s & 3];
}

// Where a chunk's operands live: first token, length, record index.
struct ChunkRef {
  long long c0;
  int c;
  int rec;
};

// Per-thread, chunk-invariant pieces of the operand copies.
struct DmaLane {
  int row;          // first K / Q / V row this lane copies (then +32 per pass)
  uint32_t kq_col;   // byte offset of its K / Q source chunk inside the row
  uint32_t v_col;    // byte offset of its V source chunk inside the row
};

// Issue the copies of one chunk's operands into buffer P.  The copies are
// asynchronous; the barrier that ends the current chunk waits for them.
template <int P>
__device__ __forceinline__ void dma_chunk(ConsumerSmem& sm, const ChunkRef& cr, const DmaLane& dl,
                                          int w, int lane, int h, int hq,
                                          const uint16_t* __restrict__ q,
                                          const uint16_t* __restrict__ k,
                                          const uint16_t* __restrict__ v,
                                          const uint16_t* __restrict__ ws_frag,
                                          const float* __restrict__ ws_gam) {
  const int cm1 = cr.c - 1;
  const size_t qk0 = (static_cast<size_t>(cr.c0) * kQKHeads + hq) * kDim;
  const char* kb = reinterpret_cast<const char*>(k + qk0);
  const char* qb = reinterpret_cast<const char*>(q + qk0);
  const char* vb = reinterpret_cast<const char*>(v + (static_cast<size_t>(cr.c0) * kVHeads + h) * kDim);
  // each wave copies 4 rows (1 KB) per pass; 8 waves x 2 passes = 64 rows
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t row = static_cast<uint32_t>(min(dl.row + 32 * j, cm1));
    const uint32_t off = row * (kQKHeads * kDim * 2) + dl.kq_col;
    dma16(kb + off, &sm.ks[P][32 * j + 4 * w][0]);
    dma16(qb + off, &sm.qs[P][32 * j + 4 * w][0]);
    dma16(vb + row * (kVHeads * kDim * 2) + dl.v_col, &sm.vs[P][32 * j + 4 * w][0]);
  }
  const size_t rh = static_cast<size_t>(cr.rec) * kVHeads + h;
  const char* fb = reinterpret_cast<const char*>(ws_frag + rh * 3 * kFragElems);
#pragma unroll
  for (int j = 0; j < 3; ++j)
    dma16(fb + (512 * j + 64 * w + lane) * 16, &sm.frag[P][0][0] + (512 * j + 64 * w) * 8);
  if (w == 0)   // gam and tail are contiguous (512 bytes); lanes 32..63 fill the padding
    dma16(reinterpret_cast<const char*>(ws_gam + rh * 2 * kChunk) + 16 * (lane & 31), &sm.gt[P][0]);
}

// One chunk of the recurrence for the 16-wide V tile of this wave.
//   st : S^T tile in C layout with a k order chosen for the K row reads:
//        st[kt][rr] = S[v0 + l16][kappa(kt, lg, rr)],
//        kappa(kt, lg, rr) = 32 (kt >> 1) + 8 lg + 4 (kt & 1) + rr,
//        so the 8 slots of depth chunk d, st[2d + s/4][s%4], are k = 32 d + 8 lg + s:
//        one contiguous 16-byte piece of a K / Q row.
//   orc : buffer resource over the chunk's output rows [c0, c0 + c) of this head
//         (num_records = c rows, so stores of rows t >= c are dropped by the
//         range check: no branch); ocol = byte offset of value column v0 + 4 lg.
template <int P>
__device__ __forceinline__ void consumer_chunk(const ConsumerSmem& sm, int c, f32x4 (&st)[8], int w,
                                               int lane, float scale, __amdgpu_buffer_rsrc_t orc,
                                               uint32_t ocol) {
  const int l16 = lane & 15, lg = lane >> 4;
  f32x4 gam[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) gam[m] = *reinterpret_cast<const f32x4*>(&sm.gt[P][16 * m + 4 * lg]);
  const float gam_c = sm.gt[P][c - 1];

  // ---- X = K S^T (rows t), Y^T = S Q^T (rows v); S as single bf16 ----
  bf16x8 sb[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float x[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) x[s] = st[2 * d + (s >> 2)][s & 3];
    sb[d] = round_frag(x);
  }
  const int rsw = kq_swz(l16);           // row t = 16 m + l16 has t & 15 == l16
  f32x4 X[4], YT[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    X[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    YT[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int at = 8 * ((4 * d + lg) ^ rsw);
      const bf16x8 ka = *reinterpret_cast<const bf16x8*>(&sm.ks[P][16 * m + l16][at]);
      const bf16x8 qa = *reinterpret_cast<const bf16x8*>(&sm.qs[P][16 * m + l16][at]);
      X[m] = mfma16(ka, sb[d], X[m]);
      YT[m] = mfma16(sb[d], qa, YT[m]);
    }
  }

  // ---- R = V - gam X (V columns by transposed LDS reads), Delta = Tb R ----
  // lane (lg, l16) addresses row 16m + 4lg + l16/4, columns 16w + 4(l16 & 3) .. +3
  const int vrow = 4 * lg + (l16 >> 2);
  const int vat = 8 * ((2 * w + ((l16 & 3) >> 1)) ^ v_swz(vrow)) + 4 * (l16 & 1);
  f32x4 Rt[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const u32x2 vw = lds_tr16(&sm.vs[P][16 * m + vrow][vat]);
    const float vv[4] = {bf_lo(vw.x), bf_hi(vw.x), bf_lo(vw.y), bf_hi(vw.y)};
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) Rt[m][rr] = vv[rr] - gam[m][rr] * X[m][rr];
  }
  bf16x8 rh[2], rl[2];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    float x[8];
    gather_slots(Rt, d, x);
    split_frag(x, rh[d], rl[d]);
  }
  f32x4 D[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    D[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int fo = ((m * 2 + d) * 64 + lane) * 8;
      const bf16x8 th = *reinterpret_cast<const bf16x8*>(&sm.frag[P][0][fo]);
      const bf16x8 tl = *reinterpret_cast<const bf16x8*>(&sm.frag[P][1][fo]);
      D[m] = mfma16(th, rh[d], D[m]);
      D[m] = mfma16(th, rl[d], D[m]);
      D[m] = mfma16(tl, rh[d], D[m]);
    }
  }

  // ---- Delta as bf16 (output) and Delta' = tail Delta as hi + lo (state) ----
  bf16x8 dob[2], dh[2], dl[2];
  {
    f32x4 Dt[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
      Dt[m] = D[m] * *reinterpret_cast<const f32x4*>(&sm.gt[P][kChunk + 16 * m + 4 * lg]);
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      float x[8];
      gather_slots(D, d, x);
      dob[d] = round_frag(x);
      gather_slots(Dt, d, x);
      split_frag(x, dh[d], dl[d]);
    }
  }

  // ---- O^T = scale (Y^T diag(gam) + Delta^T Aqk^T): lane (lg, l16) holds token
  //      16m + l16, value columns 4lg .. 4lg+3 -> one 8-byte store ----
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    f32x4 OT = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 2; ++d)
      OT = mfma16(dob[d], *reinterpret_cast<const bf16x8*>(&sm.frag[P][2][((m * 2 + d) * 64 + lane) * 8]), OT);
    const int t = 16 * m + l16;
    const float sg = scale * sm.gt[P][t];
    const u32x2 pk = {pack_bf2(sg * YT[m][0] + scale * OT[0], sg * YT[m][1] + scale * OT[1]),
                      pack_bf2(sg * YT[m][2] + scale * OT[2], sg * YT[m][3] + scale * OT[3])};
    __builtin_amdgcn_raw_buffer_store_b64(pk, orc, static_cast<uint32_t>(t) * (kVHeads * kDim * 2) + ocol, 0, 0);
  }

  // ---- S^T <- gam_c S^T + K^T Delta' (K^T fragments by transposed reads) ----
  // Tile kt, row i of the A operand is k = kappa(kt, i/4, i%4).  Lane sl of
  // group lg addresses K[t][k0 .. k0+3], t = perm_depth(d, lg, sl/4) (+16 for
  // slots 4..7), k0 = 32 (kt >> 1) + 8 (sl & 3) + 4 (kt & 1).
  const int sl = l16;
  const int tsw = kq_swz(4 * lg + (sl >> 2));   // t & 15 for both row sets
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    f32x4 acc = st[kt] * gam_c;
    const int at = 8 * ((4 * (kt >> 1) + (sl & 3)) ^ tsw) + 4 * (kt & 1);
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int ta = perm_depth(d, lg, sl >> 2);
      const u32x2 a0 = lds_tr16(&sm.ks[P][ta][at]);
      const u32x2 a1 = lds_tr16(&sm.ks[P][ta + 16][at]);
      const bf16x8 kta = join_frag(a0, a1);
      acc = mfma16(kta, dh[d], acc);
      acc = mfma16(kta, dl[d], acc);
    }
    st[kt] = acc;
  }
}

// One work-group per CU by design: 146 KB of double-buffered chunk operands,
// two waves per SIMD.
__global__ __launch_bounds__(kConsumerThreads)
void consumer_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                     const uint16_t* __restrict__ v, const float* __restrict__ state,
                     const void* __restrict__ cu, int is64, long long T, int R, float scale,
                     const int* __restrict__ rec_start, const uint16_t* __restrict__ ws_frag,
                     const float* __restrict__ ws_gam, uint16_t* __restrict__ out,
                     float* __restrict__ new_state) {
  __shared__ ConsumerSmem sm;
  // XCD-aware mapping (XCD = linear id % 8): v-head h runs on XCD h, where its
  // prepass records were written.
  const int bid = blockIdx.x;
  const int h = bid & 7;
  const int s = bid >> 3;
  const int hq = h / kGva;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int vcol = 16 * w;                       // first value row of this wave's tile

  long long t0, t1;
  seq_bounds(cu, is64, s, T, t0, t1);
  // state tile in the kappa k order (see consumer_chunk)
  const size_t st_off = ((static_cast<size_t>(s) * kVHeads + h) * kDim + vcol + l16) * kDim + 8 * lg;
  auto kappa0 = [](int kt) { return 32 * (kt >> 1) + 4 * (kt & 1); };
  if (t1 <= t0) {   // empty sequence: the reference leaves new_state zero
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      *reinterpret_cast<f32x4*>(new_state + st_off + kappa0(kt)) = f32x4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  const int rec0 = rec_start[s];
  const long long nchunks = (t1 - t0 + kChunk - 1) / kChunk;
  // chunks whose records exist (overlapping cu_seqlens can exhaust the capacity)
  const long long nvalid = rec0 >= R ? 0 : min(nchunks, static_cast<long long>(R - rec0));
  auto chunk_ref = [&](long long idx) {
    const long long c0 = t0 + idx * kChunk;
    return ChunkRef{c0, static_cast<int>(min(static_cast<long long>(kChunk), t1 - c0)),
                    rec0 + static_cast<int>(idx)};
  };

  f32x4 st[8];
  if (state != nullptr) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) st[kt] = *reinterpret_cast<const f32x4*>(state + st_off + kappa0(kt));
  } else {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  DmaLane dl;
  {
    const int r = 4 * w + (lane >> 4);     // + 32 j keeps r & 15
    dl.row = r;
    dl.kq_col = 16u * static_cast<uint32_t>((lane & 15) ^ kq_swz(r));
    dl.v_col = 16u * static_cast<uint32_t>((lane & 15) ^ v_swz(r));
  }
  const uint32_t ocol = 2u * static_cast<uint32_t>(vcol + 4 * lg);
  auto out_rsrc = [&](const ChunkRef& cr) {
    return __builtin_amdgcn_make_buffer_rsrc(out + (static_cast<size_t>(cr.c0) * kVHeads + h) * kDim, 0,
                                             cr.c * (kVHeads * kDim * 2), 0x00020000);
  };

  if (nvalid > 0) {
    // Chunk i computes from buffer i & 1 while the copies of chunk i+1 into the
    // other buffer are in flight; the barrier closing chunk i waits for them
    // (and frees buffer i & 1 for chunk i+2).
    dma_chunk<0>(sm, chunk_ref(0), dl, w, lane, h, hq, q, k, v, ws_frag, ws_gam);
    __syncthreads();
    for (long long i = 0; i < nvalid; i += 2) {
      {
        if (i + 1 < nvalid) dma_chunk<1>(sm, chunk_ref(i + 1), dl, w, lane, h, hq, q, k, v, ws_frag, ws_gam);
        const ChunkRef cr = chunk_ref(i);
        consumer_chunk<0>(sm, cr.c, st, w, lane, scale, out_rsrc(cr), ocol);
        __syncthreads();
      }
      if (i + 1 < nvalid) {
        if (i + 2 < nvalid) dma_chunk<0>(sm, chunk_ref(i + 2), dl, w, lane, h, hq, q, k, v, ws_frag, ws_gam);
        const ChunkRef cr = chunk_ref(i + 1);
        consumer_chunk<1>(sm, cr.c, st, w, lane, scale, out_rsrc(cr), ocol);
        __syncthreads();
      }
    }
  }

#pragma unroll
  for (int kt = 0; kt < 8; ++kt) *reinterpret_cast<f32x4*>(new_state + st_off + kappa0(kt)) = st[kt];
}

}  // namespace gdn

extern "C" size_t gdn_prefill_workspace_bytes(int num_seqs, long long total_tokens) {
  if (num_seqs < 0 || total_tokens < 0) return 0;
  return gdn::ws_layout(num_seqs, total_tokens).total;
}

extern "C" int gdn_prefill_fwd(const void* q, const void* k, const void* v, const float* state,
                               const float* A_log, const void* a, const float* dt_bias,
                               const void* b, const void* cu_seqlens, int cu_seqlens_is_int64,
                               int num_seqs, long long total_tokens, float scale, void* output,
                               float* new_state, void* workspace, size_t workspace_bytes,
                               void* stream) {
  using namespace gdn;
  if (num_seqs < 0 || total_tokens < 0) return GDN_ERR_INVALID_ARGUMENT;
  if (num_seqs == 0) return GDN_OK;
  if (!cu_seqlens || !new_state || !workspace || !A_log || !dt_bias)
    return GDN_ERR_INVALID_ARGUMENT;
  if (total_tokens > 0 && (!q || !k || !v || !a || !b || !output)) return GDN_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) & 15u) return GDN_ERR_UNALIGNED;
  if ((reinterpret_cast<uintptr_t>(state) | reinterpret_cast<uintptr_t>(new_state)) & 15u)
    return GDN_ERR_UNALIGNED;
  if (reinterpret_cast<uintptr_t>(workspace) & 255u) return GDN_ERR_UNALIGNED;
  if (state != nullptr && state == new_state) return GDN_ERR_ALIASING;
  const long long R = max_records(num_seqs, total_tokens);
  if (R * kVHeads > 0x7fffffffLL || static_cast<long long>(num_seqs) * kVHeads > 0x7fffffffLL)
    return GDN_ERR_INVALID_ARGUMENT;
  const WsLayout L = ws_layout(num_seqs, total_tokens);
  if (workspace_bytes < L.total) return GDN_ERR_WORKSPACE_TOO_SMALL;
  if (!(scale > 0.0f) && !(scale < 0.0f)) scale = 0.08838834764831845f;

  char* ws = static_cast<char*>(workspace);
  auto* frag = reinterpret_cast<uint16_t*>(ws + L.frag_off);
  auto* gam = reinterpret_cast<float*>(ws + L.gam_off);
  auto* rec_start = reinterpret_cast<int*>(ws + L.start_off);
  auto* recs = reinterpret_cast<int4*>(ws + L.rec_off);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  const auto* ab = static_cast<const uint16_t*>(a);
  const auto* bb = static_cast<const uint16_t*>(b);
  auto* ob = static_cast<uint16_t*>(output);

  plan_kernel<<<dim3(1), dim3(kPlanThreads), 0, st>>>(cu_seqlens, cu_seqlens_is_int64, num_seqs,
                                                      total_tokens, static_cast<int>(R), rec_start,
                                                      recs);
  prepass_kernel<<<dim3(static_cast<unsigned>(R * kVHeads)), dim3(256), 0, st>>>(
      qb, kb, A_log, ab, dt_bias, bb, recs, frag, gam);
  consumer_kernel<<<dim3(static_cast<unsigned>(num_seqs) * kVHeads), dim3(kConsumerThreads), 0, st>>>(
      qb, kb, vb, state, cu_seqlens, cu_seqlens_is_int64, total_tokens, static_cast<int>(R), scale,
      rec_start, frag, gam, ob, new_state);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? GDN_OK : static_cast<int>(err);
}
