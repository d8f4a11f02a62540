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
//              and the packed MFMA operands Tb (bf16 hi+lo), Aqk (bf16),
//              K^T (bf16) plus gam / tail, written to the workspace.
//   consumer : one work-group (4 waves) per (seq, v-head, 16-wide V tile),
//              sequential over the sequence's chunks, state tile in registers.
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
constexpr int kBV = 16;                      // consumer V tile
constexpr int kVTiles = kDim / kBV;          // 8
constexpr int kFragElems = 4096;             // 64x64 bf16 operand in fragment order
constexpr int kKTElems = kDim * kChunk;      // 128x64 bf16 K^T in fragment order

// ---- workspace layout -------------------------------------------------------
struct WsLayout {
  size_t frag_off;     // bf16 [R][8][3][4096]   (Tb hi, Tb lo, Aqk)
  size_t gam_off;      // f32  [R][8][2][64]     (gam, tail)
  size_t kt_off;       // bf16 [R][4][8192]      (K^T)
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
  L.kt_off = off;    off = align256(off + R * kQKHeads * kKTElems * sizeof(uint16_t));
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
// prepass: chunk-local WY terms for one (record, v-head)
// ============================================================================
constexpr int kQKRow = 136;   // bf16 per LDS row of K / Q (128 + 8 pad, 16-byte aligned)
constexpr int kMRow = 68;     // floats per LDS row of the 64x64 fp32 matrices

struct __align__(16) PrepassSmem {
  uint16_t kk[kChunk][kQKRow];
  uint16_t qq[kChunk][kQKRow];
  float nmat[kChunk][kMRow];      // strict lower beta_t rho K K^T
  float tmat[kChunk][kMRow];      // first Aqk, then T = (I + N)^{-1}
  float pscr[4][16][17];          // per-wave 16x16 product scratch
  float lgam[kChunk];             // Gam_t / ln 2 (log2 cumulative decay)
  float beta[kChunk];
};

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 lds_frag(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

// j-th lower 16x16 tile (mi >= ni) of a 4x4 tile grid, row by row:
// (0,0) (1,0) (1,1) (2,0) (2,1) (2,2) (3,0) (3,1) (3,2) (3,3).
__device__ __forceinline__ void lower_tile(int j, int& mi, int& ni) {
  mi = j >= 6 ? 3 : (j >= 3 ? 2 : (j >= 1 ? 1 : 0));
  ni = j - mi * (mi + 1) / 2;
}

// P[rows 4(l/16)..+3][col l%16] = sum_u A[r][u] * B[u][c] for 16x16 blocks in LDS.
__device__ __forceinline__ void block_mma_acc(float (&acc)[4], const float* A, int lda,
                                              const float* B, int ldb, int r0, int c) {
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const float bv = B[u * ldb + c];
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[a] = fmaf(A[(r0 + a) * lda + u], bv, acc[a]);
  }
}

__global__ __launch_bounds__(256) void prepass_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const int4* __restrict__ recs, uint16_t* __restrict__ ws_frag,
    float* __restrict__ ws_gam, uint16_t* __restrict__ ws_kt) {
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
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int lg = lane >> 4;

  // ---- K, Q rows of the chunk into LDS (rows >= c zero) ----
  // All loads are issued before any is used (clamped rows, zeroed by select)
  // so the work-group pays one memory round trip, not one per row group.
  {
    uint4 kv[4], qv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int idx = tid + 256 * j;
      const int row = min(idx >> 4, c - 1);
      const size_t off = ((t0 + row) * kQKHeads + hq) * kDim + (idx & 15) * 8;
      kv[j] = *reinterpret_cast<const uint4*>(k + off);
      qv[j] = *reinterpret_cast<const uint4*>(q + off);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int idx = tid + 256 * j;
      const int row = idx >> 4;
      const uint4 z = make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(&sm.kk[row][(idx & 15) * 8]) = row < c ? kv[j] : z;
      *reinterpret_cast<uint4*>(&sm.qq[row][(idx & 15) * 8]) = row < c ? qv[j] : z;
    }
  }

  // ---- gates (wave 0): Gam_t inclusive scan of log g, beta ----
  if (wave == 0) {
    const int t = lane;
    const size_t gi = (t0 + min(t, c - 1)) * kVHeads + h;
    const float a_t = bf2f(a[gi]), b_t = bf2f(b[gi]);
    // clamp: g = e^-100 is already 0 to fp32 working precision, and a finite
    // floor keeps Gam finite (no -inf - -inf) for absurd gate inputs
    // log2 of the decay (Gam kept in log2 units so every ratio is one v_exp_f32)
    const float lgv = t < c ? fmaxf(log_decay(A_log[h], a_t, dt_bias[h]), -100.0f) * kLog2e : 0.0f;
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

  // ---- K K^T and Q K^T lower tiles on MFMA; masked gate weighting ----
  for (int job = wave; job < 20; job += 4) {
    const int which = job / 10;                  // 0: K K^T -> N, 1: Q K^T -> Aqk
    int mi, ni;
    lower_tile(job % 10, mi, ni);
    const uint16_t(*lhs)[kQKRow] = which ? sm.qq : sm.kk;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const bf16x8 av = lds_frag(&lhs[16 * mi + l16][32 * d + 8 * lg]);
      const bf16x8 bv = lds_frag(&sm.kk[16 * ni + l16][32 * d + 8 * lg]);
      acc = mfma16(av, bv, acc);
    }
    const int col = 16 * ni + l16;
    const float gcol = sm.lgam[col];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int row = 16 * mi + 4 * lg + rr;
      const float rho = col <= row ? fast_exp2(sm.lgam[row] - gcol) : 0.0f;
      if (which == 0) {
        sm.nmat[row][col] = col < row ? sm.beta[row] * rho * acc[rr] : 0.0f;
      } else {
        sm.tmat[row][col] = rho * acc[rr];
      }
    }
  }
  __syncthreads();

  // ---- pack Aqk (bf16, fragment order; upper triangle zero) ----
  uint16_t* frag = ws_frag + (static_cast<size_t>(r) * kVHeads + h) * 3 * kFragElems;
  for (int qi = tid; qi < 512; qi += 256) {
    const int m = qi >> 7, d = (qi >> 6) & 1, l = qi & 63;
    const int row = 16 * m + (l & 15);
    const int dep = 32 * d + 8 * (l >> 4);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i0 = dep + 2 * j, i1 = i0 + 1;
      const float x0 = i0 <= row ? sm.tmat[row][i0] : 0.0f;
      const float x1 = i1 <= row ? sm.tmat[row][i1] : 0.0f;
      w[j] = pack_bf2(x0, x1);
    }
    *reinterpret_cast<uint4*>(frag + 2 * kFragElems + qi * 8) = make_uint4(w[0], w[1], w[2], w[3]);
  }

  // ---- K^T in fragment order (once per q/k head, by the even v-head) ----
  if ((h & 1) == 0) {
    uint16_t* kt = ws_kt + (static_cast<size_t>(r) * kQKHeads + hq) * kKTElems;
    for (int qi = tid; qi < 1024; qi += 256) {
      const int m = qi >> 7, d = (qi >> 6) & 1, l = qi & 63;
      const int kcol = 16 * m + (l & 15);
      const int t = 32 * d + 8 * (l >> 4);
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = static_cast<uint32_t>(sm.kk[t + 2 * j][kcol]) |
               (static_cast<uint32_t>(sm.kk[t + 2 * j + 1][kcol]) << 16);
      *reinterpret_cast<uint4*>(kt + qi * 8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  __syncthreads();   // Aqk consumed from tmat; tmat is free for T

  // ---- T = (I + N)^{-1}: diagonal 16x16 blocks by forward substitution ----
  if (lane < 16) {
    const int base = 16 * wave;
    const int j = lane;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = (i == j) ? 1.0f : 0.0f;
#pragma unroll
      for (int m2 = 0; m2 < i; ++m2) acc = fmaf(-sm.nmat[base + i][base + m2], x[m2], acc);
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sm.tmat[base + i][base + j] = x[i];
  }
  __syncthreads();

  // ---- off-diagonal blocks: T_ij = -T_ii sum_{m=j}^{i-1} N_im T_mj, by distance ----
  const int r0 = 4 * lg;
  for (int dist = 1; dist < 4; ++dist) {
    const bool active = wave < 4 - dist;
    const int bj = wave, bi = wave + dist;
    if (active) {
      float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int bm = bj; bm < bi; ++bm)
        block_mma_acc(p, &sm.nmat[16 * bi][16 * bm], kMRow, &sm.tmat[16 * bm][16 * bj], kMRow,
                      r0, l16);
#pragma unroll
      for (int aa = 0; aa < 4; ++aa) sm.pscr[wave][r0 + aa][l16] = p[aa];
    }
    __syncthreads();
    if (active) {
      float t4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      block_mma_acc(t4, &sm.tmat[16 * bi][16 * bi], kMRow, &sm.pscr[wave][0][0], 17, r0, l16);
#pragma unroll
      for (int aa = 0; aa < 4; ++aa) sm.tmat[16 * bi + r0 + aa][16 * bj + l16] = -t4[aa];
    }
    __syncthreads();
  }

  // ---- pack Tb = T diag(beta) as bf16 hi + lo (fragment order) ----
  for (int qi = tid; qi < 512; qi += 256) {
    const int m = qi >> 7, d = (qi >> 6) & 1, l = qi & 63;
    const int row = 16 * m + (l & 15);
    const int dep = 32 * d + 8 * (l >> 4);
    uint32_t wh[4], wl[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i0 = dep + 2 * j, i1 = i0 + 1;
      const float x0 = i0 <= row ? sm.tmat[row][i0] * sm.beta[i0] : 0.0f;
      const float x1 = i1 <= row ? sm.tmat[row][i1] * sm.beta[i1] : 0.0f;
      const uint16_t h0 = f2bf(x0), h1 = f2bf(x1);
      wh[j] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
      wl[j] = pack_bf2(x0 - bf2f(h0), x1 - bf2f(h1));
    }
    *reinterpret_cast<uint4*>(frag + qi * 8) = make_uint4(wh[0], wh[1], wh[2], wh[3]);
    *reinterpret_cast<uint4*>(frag + kFragElems + qi * 8) = make_uint4(wl[0], wl[1], wl[2], wl[3]);
  }
}

// ============================================================================
// consumer: sequential chunk loop for one (seq, v-head, 16-wide V tile)
// ============================================================================
constexpr int kSRow = 136;    // bf16 per LDS row of S (v-major, k contiguous)
constexpr int kTRow = 72;     // bf16 per LDS row of the [v][t] operands

struct __align__(16) ConsumerSmem {
  // Wave-private staging of the chunk's K / Q rows (16 rows per wave, 16-byte
  // k-chunks XOR-swizzled by row so fragment reads and row writes are both
  // bank-conflict free) and of its V rows (16 rows x 16 values).
  uint16_t kq[4][2][16][kDim];
  uint16_t vs[4][16][kBV];
  uint16_t s_bf[kBV][kSRow];      // S tile as bf16, [v][k]
  uint16_t r_hi[kBV][kTRow];      // R = V - gam K S^T, [v][t]
  uint16_t r_lo[kBV][kTRow];
  uint16_t d_o[kBV][kTRow];       // Delta (bf16) for the output
  uint16_t d_hi[kBV][kTRow];      // tail * Delta, hi / lo, for the state update
  uint16_t d_lo[kBV][kTRow];
};

__device__ __forceinline__ bf16x8 gload_frag(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

__device__ __forceinline__ void split_store4(uint16_t* hi_dst, uint16_t* lo_dst, const float (&x)[4]) {
  uint16_t hv[4];
  float lv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hv[i] = f2bf(x[i]);
    lv[i] = x[i] - bf2f(hv[i]);
  }
  *reinterpret_cast<uint2*>(hi_dst) =
      make_uint2(static_cast<uint32_t>(hv[0]) | (static_cast<uint32_t>(hv[1]) << 16),
                 static_cast<uint32_t>(hv[2]) | (static_cast<uint32_t>(hv[3]) << 16));
  *reinterpret_cast<uint2*>(lo_dst) = make_uint2(pack_bf2(lv[0], lv[1]), pack_bf2(lv[2], lv[3]));
}

__device__ __forceinline__ void store_bf4(uint16_t* dst, const float (&x)[4]) {
  *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf2(x[0], x[1]), pack_bf2(x[2], x[3]));
}

// Per-lane operands of one chunk step, loaded one chunk ahead so that the
// global-memory latency overlaps the previous chunk's MFMA/LDS chain.
struct ChunkOps {
  u32x4 kr[4], qr[4];        // K, Q rows 16w + 4i + lane/16, 16-byte k-chunk lane%16
  bf16x8 th[2], tl[2];       // Tb hi / lo fragments (rows 16w.., depth 32d..)
  bf16x8 aq[2];              // Aqk fragments
  bf16x8 kt[2][2];           // K^T fragments for k tiles 2w + i
  f32x4 gam, tail;           // gam_t, tail_t for t = 16w + 4lg + rr
  u32x2 vr;                  // V row 16w + lane/4, values v0 + 4(lane%4) .. +3
  float gam_c;
  int c;                     // chunk length
  long long c0;              // first token
};

// Where a chunk's operands live: first token, length, record index.
struct ChunkRef {
  long long c0;
  int c;
  int rec;
};

// Operand loads of one chunk, in three parts issued at different points of the
// previous steps so that the vector-memory pipe streams them while the MFMA
// chain runs (issued as one burst they stall the issuing wave for thousands
// of cycles).  Rows past the chunk end are clamped to the last valid row
// instead of being masked: unconditional loads keep the prefetch free of wait
// points, and the duplicate rows are harmless because gam, Tb and the V mask
// zero R, Delta and every state contribution for t >= c, and their outputs are
// never stored.
template <int PART>
__device__ __forceinline__ void load_chunk_part(
    ChunkOps& o, const ChunkRef& r, int h, int hq, int v0, int w, int lane,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ ws_frag,
    const float* __restrict__ ws_gam, const uint16_t* __restrict__ ws_kt) {
  const int l16 = lane & 15, lg = lane >> 4;
  if constexpr (PART == 0) {
    // 16 lanes read one 256-byte head row, so each load covers 4 whole rows
    o.c0 = r.c0;
    o.c = r.c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = min(16 * w + 4 * i + lg, r.c - 1);
      const size_t off = ((r.c0 + row) * kQKHeads + hq) * kDim + 8 * l16;
      o.kr[i] = *reinterpret_cast<const u32x4*>(k + off);
      o.qr[i] = *reinterpret_cast<const u32x4*>(q + off);
    }
    {
      const int row = min(16 * w + (lane >> 2), r.c - 1);   // masked to 0 for t >= c where used
      o.vr = *reinterpret_cast<const u32x2*>(v + ((r.c0 + row) * kVHeads + h) * kDim + v0 +
                                             4 * (lane & 3));
    }
  } else if constexpr (PART == 1) {
    const uint16_t* frag = ws_frag + (static_cast<size_t>(r.rec) * kVHeads + h) * 3 * kFragElems;
    const float* gp = ws_gam + (static_cast<size_t>(r.rec) * kVHeads + h) * 2 * kChunk;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int fo = ((w * 2 + d) * 64 + lane) * 8;
      o.th[d] = gload_frag(frag + fo);
      o.tl[d] = gload_frag(frag + kFragElems + fo);
    }
    const int tb = 16 * w + 4 * lg;
    o.gam = *reinterpret_cast<const f32x4*>(gp + tb);
    o.tail = *reinterpret_cast<const f32x4*>(gp + kChunk + tb);
    o.gam_c = gp[r.c - 1];
  } else {
    const uint16_t* frag = ws_frag + (static_cast<size_t>(r.rec) * kVHeads + h) * 3 * kFragElems;
    const uint16_t* kt = ws_kt + (static_cast<size_t>(r.rec) * kQKHeads + hq) * kKTElems;
#pragma unroll
    for (int d = 0; d < 2; ++d)
      o.aq[d] = gload_frag(frag + 2 * kFragElems + ((w * 2 + d) * 64 + lane) * 8);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int d = 0; d < 2; ++d)
        o.kt[i][d] = gload_frag(kt + (((2 * w + i) * 2 + d) * 64 + lane) * 8);
  }
}

// Raw K / Q / V rows of a chunk -> this wave's LDS staging area.
__device__ __forceinline__ void stage_rows(const ChunkOps& o, ConsumerSmem& sm, int w, int lane) {
  const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * i + lg;
    *reinterpret_cast<u32x4*>(&sm.kq[w][0][row][8 * (l16 ^ row)]) = o.kr[i];
    *reinterpret_cast<u32x4*>(&sm.kq[w][1][row][8 * (l16 ^ row)]) = o.qr[i];
  }
  *reinterpret_cast<u32x2*>(&sm.vs[w][lane >> 2][4 * (lane & 3)]) = o.vr;
}

// A fragment d (k = 32d + 8lg .. +7 of row l16) of the staged K (m = 0) or Q (m = 1).
__device__ __forceinline__ bf16x8 staged_frag(const ConsumerSmem& sm, int w, int m, int d,
                                              int l16, int lg) {
  return *reinterpret_cast<const bf16x8*>(&sm.kq[w][m][l16][8 * ((4 * d + lg) ^ l16)]);
}

// Pointers and coordinates every chunk load of one consumer wave shares.
struct LoadCtx {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* ws_frag;
  const float* ws_gam;
  const uint16_t* ws_kt;
  int h, hq, v0, w, lane;
};

template <int PART>
__device__ __forceinline__ void load_part(ChunkOps& o, const ChunkRef& r, const LoadCtx& L) {
  load_chunk_part<PART>(o, r, L.h, L.hq, L.v0, L.w, L.lane, L.q, L.k, L.v, L.ws_frag, L.ws_gam,
                        L.ws_kt);
}

__device__ __forceinline__ void load_chunk_ops(ChunkOps& o, const ChunkRef& r, const LoadCtx& L) {
  load_part<0>(o, r, L);
  load_part<1>(o, r, L);
  load_part<2>(o, r, L);
}

// One chunk step of the consumer for wave w: reads the state tile from LDS
// (bf16) and its fp32 C-layout registers st, writes this chunk's outputs and
// the advanced state.  Three work-group barriers.
// The operands of chunk `pre` are loaded into `nxt` in three parts between
// the stages; the raw rows of the following chunk (`mid`) replace this
// chunk's in the wave's staging area once its fragments are in registers.
__device__ __forceinline__ void consumer_step(const ChunkOps& cur, const ChunkOps& mid, ChunkOps& nxt,
                                              const ChunkRef& pre,
                                              const LoadCtx& L, f32x4 (&st)[2], ConsumerSmem& sm,
                                              int h, int v0, int w, int l16, int lg, float scale,
                                              uint16_t* __restrict__ out) {
  const int c = cur.c;
  const long long c0 = cur.c0;
  // ---- stage 1: X = K S^T, Y = Q S^T for token rows 16w .. 16w+15 ----
  f32x4 X = {0.f, 0.f, 0.f, 0.f}, Y = {0.f, 0.f, 0.f, 0.f};
  bf16x8 ka[4], qa[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    ka[d] = staged_frag(sm, w, 0, d, l16, lg);
    qa[d] = staged_frag(sm, w, 1, d, l16, lg);
  }
  uint16_t vv[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) vv[rr] = sm.vs[w][4 * lg + rr][l16];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const bf16x8 sb = lds_frag(&sm.s_bf[l16][32 * d + 8 * lg]);
    X = mfma16(ka[d], sb, X);
    Y = mfma16(qa[d], sb, Y);
  }
  stage_rows(mid, sm, w, L.lane);
  load_part<0>(nxt, pre, L);

  // ---- stage 2: R = V - gam X (hi/lo to LDS), Delta = Tb R ----
  {
    float rv[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const float vf = (16 * w + 4 * lg + rr < c) ? bf2f(vv[rr]) : 0.0f;
      rv[rr] = vf - cur.gam[rr] * X[rr];
    }
    split_store4(&sm.r_hi[l16][16 * w + 4 * lg], &sm.r_lo[l16][16 * w + 4 * lg], rv);
  }
  __syncthreads();
  f32x4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const bf16x8 rh = lds_frag(&sm.r_hi[l16][32 * d + 8 * lg]);
    const bf16x8 rl = lds_frag(&sm.r_lo[l16][32 * d + 8 * lg]);
    D = mfma16(cur.th[d], rh, D);
    D = mfma16(cur.th[d], rl, D);
    D = mfma16(cur.tl[d], rh, D);
  }
  load_part<1>(nxt, pre, L);

  // ---- stage 3: Delta to LDS; O = scale (gam Y + Aqk Delta) ----
  {
    const float dv[4] = {D[0], D[1], D[2], D[3]};
    float dt[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) dt[rr] = cur.tail[rr] * D[rr];
    store_bf4(&sm.d_o[l16][16 * w + 4 * lg], dv);
    split_store4(&sm.d_hi[l16][16 * w + 4 * lg], &sm.d_lo[l16][16 * w + 4 * lg], dt);
  }
  __syncthreads();
  {
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const bf16x8 db = lds_frag(&sm.d_o[l16][32 * d + 8 * lg]);
      O = mfma16(cur.aq[d], db, O);
    }
    load_part<2>(nxt, pre, L);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int t = 16 * w + 4 * lg + rr;
      if (t < c) {
        const float o = scale * (cur.gam[rr] * Y[rr] + O[rr]);
        out[((c0 + t) * kVHeads + h) * kDim + v0 + l16] = f2bf(o);
      }
    }
  }

  // ---- stage 4: S^T <- gam_c S^T + K^T Delta' for this wave's k rows ----
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    f32x4 acc = st[i] * cur.gam_c;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const bf16x8 dh = lds_frag(&sm.d_hi[l16][32 * d + 8 * lg]);
      const bf16x8 dl = lds_frag(&sm.d_lo[l16][32 * d + 8 * lg]);
      acc = mfma16(cur.kt[i][d], dh, acc);
      acc = mfma16(cur.kt[i][d], dl, acc);
    }
    st[i] = acc;
    const float x[4] = {acc[0], acc[1], acc[2], acc[3]};
    store_bf4(&sm.s_bf[l16][32 * w + 16 * i + 4 * lg], x);
  }
  __syncthreads();
}

// One work-group per CU by design (4 waves, one per SIMD): the register ring
// of chunk operands needs the whole 512-entry VGPR+AGPR file of a SIMD.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void consumer_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ state,
    const void* __restrict__ cu, int is64, long long T, int R, float scale,
    const int* __restrict__ rec_start, const uint16_t* __restrict__ ws_frag,
    const float* __restrict__ ws_gam, const uint16_t* __restrict__ ws_kt,
    uint16_t* __restrict__ out, float* __restrict__ new_state) {
  __shared__ ConsumerSmem sm;
  // XCD-aware mapping: work-groups are dispatched round-robin over the 8 XCDs
  // (XCD = linear id % 8).  The 8 V tiles of one (seq, v-head) read identical
  // chunk operands, so they are given ids that are equal mod 8: they share one
  // XCD's L2, and v-head h always lands on XCD h (where its prepass ran).
  const int bid = blockIdx.x;
  const int grp = (bid / (kVHeads * kVTiles)) * kVHeads + (bid % kVHeads);   // s * 8 + h
  const int vt = (bid / kVHeads) % kVTiles;
  const int s = grp / kVHeads;
  const int h = grp % kVHeads;
  const int hq = h / kGva;
  const int v0 = vt * kBV;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int lg = lane >> 4;

  long long t0, t1;
  seq_bounds(cu, is64, s, T, t0, t1);

  // State tile, transposed view S^T[k][v] in MFMA C layout: this wave owns
  // k = 32w + 16i + 4lg + rr (i < 2, rr < 4) for v = v0 + l16.
  float* ns_base = new_state + (static_cast<size_t>(s) * kVHeads + h) * kHeadState +
                   static_cast<size_t>(v0 + l16) * kDim;
  if (t1 <= t0) {   // empty sequence: the reference leaves new_state zero
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<f32x4*>(ns_base + 32 * w + 16 * i + 4 * lg) = f32x4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  const int rec0 = rec_start[s];
  const long long nchunks = (t1 - t0 + kChunk - 1) / kChunk;
  // chunks whose records exist (overlapping cu_seqlens can exhaust the capacity)
  const long long nvalid = rec0 >= R ? 0 : min(nchunks, static_cast<long long>(R - rec0));

  const LoadCtx L{q, k, v, ws_frag, ws_gam, ws_kt, h, hq, v0, w, lane};
  // chunk idx -> operand location; clamped to the last chunk so that the
  // prefetch beyond the end re-reads valid data instead of being skipped
  auto chunk_ref = [&](long long idx) {
    idx = min(idx, nvalid - 1);
    const long long c0 = t0 + idx * kChunk;
    return ChunkRef{c0, static_cast<int>(min(static_cast<long long>(kChunk), t1 - c0)),
                    rec0 + static_cast<int>(idx)};
  };
  ChunkOps bufA, bufB, bufC;
  if (nvalid > 0) {
    load_chunk_ops(bufA, chunk_ref(0), L);
    load_chunk_ops(bufB, chunk_ref(1), L);
    stage_rows(bufA, sm, w, lane);
  }
  f32x4 st[2];
  if (state != nullptr) {
    const float* s_base = state + (static_cast<size_t>(s) * kVHeads + h) * kHeadState +
                          static_cast<size_t>(v0 + l16) * kDim;
#pragma unroll
    for (int i = 0; i < 2; ++i) st[i] = *reinterpret_cast<const f32x4*>(s_base + 32 * w + 16 * i + 4 * lg);
  } else {
    st[0] = st[1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float x[4] = {st[i][0], st[i][1], st[i][2], st[i][3]};
    store_bf4(&sm.s_bf[l16][32 * w + 16 * i + 4 * lg], x);
  }
  __syncthreads();

  // Three operand buffers in a ring: chunk i + 2 is loading (spread over the
  // stages of step i) while chunk i computes.  Every consumer_step call site
  // sees the same loads in flight, so the compiler's wait counts never fall
  // back to draining everything.
  if (nvalid > 0) {
    long long ci = 0;
    for (;;) {
      consumer_step(bufA, bufB, bufC, chunk_ref(ci + 2), L, st, sm, h, v0, w, l16, lg, scale, out);
      if (++ci >= nvalid) break;
      consumer_step(bufB, bufC, bufA, chunk_ref(ci + 2), L, st, sm, h, v0, w, l16, lg, scale, out);
      if (++ci >= nvalid) break;
      consumer_step(bufC, bufA, bufB, chunk_ref(ci + 2), L, st, sm, h, v0, w, l16, lg, scale, out);
      if (++ci >= nvalid) break;
    }
  }

#pragma unroll
  for (int i = 0; i < 2; ++i) *reinterpret_cast<f32x4*>(ns_base + 32 * w + 16 * i + 4 * lg) = st[i];
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
  if (R * kVHeads > 0x7fffffffLL || static_cast<long long>(num_seqs) * kVHeads * kVTiles > 0x7fffffffLL)
    return GDN_ERR_INVALID_ARGUMENT;
  const WsLayout L = ws_layout(num_seqs, total_tokens);
  if (workspace_bytes < L.total) return GDN_ERR_WORKSPACE_TOO_SMALL;
  if (!(scale > 0.0f) && !(scale < 0.0f)) scale = 0.08838834764831845f;

  char* ws = static_cast<char*>(workspace);
  auto* frag = reinterpret_cast<uint16_t*>(ws + L.frag_off);
  auto* gam = reinterpret_cast<float*>(ws + L.gam_off);
  auto* kt = reinterpret_cast<uint16_t*>(ws + L.kt_off);
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
      qb, kb, A_log, ab, dt_bias, bb, recs, frag, gam, kt);
  consumer_kernel<<<dim3(static_cast<unsigned>(num_seqs * kVHeads * kVTiles)), dim3(256), 0, st>>>(
      qb, kb, vb, state, cu_seqlens, cu_seqlens_is_int64, total_tokens, static_cast<int>(R), scale,
      rec_start, frag, gam,
      kt, ob, new_state);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? GDN_OK : static_cast<int>(err);
}
