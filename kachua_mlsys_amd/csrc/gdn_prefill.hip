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
// Launches, all on the caller's stream, no host synchronisation:
//   plan     : (batches of more than 512 sequences only) 1 work-group: chunk
//              records, segment length and work lists from cu_seqlens.  For
//              smaller batches work-group 0 of the prepass plans and the other
//              prepass work-groups find their own records.
//   prepass  : one wave per (record, v-head), or per (record, q/k head) for
//              large batches, all records in parallel: gates, K K^T on MFMA,
//              the blocked triangular inverse (diagonal blocks by fp32 forward
//              substitution, the rest on MFMA with bf16 hi + lo operands), and
//              the packed MFMA operand Tb (fp16) plus gam / tail / Gam, written
//              to the workspace.  It never reads Q.
//   consumer : persistent work-groups.  Each chunk's Aqk is formed here, from
//              the K / Q rows in LDS, in tiles shared between the waves through
//              LDS.  Long sequences are cut into segments
//              of L chunks (L chosen by the plan); every segment runs at once,
//              segments >= 1 twice (zero initial state with the real V, and
//              identity initial state with V = 0), each run split over two
//              work-groups of 64 value rows whose chain waves carry the state
//              in MFMA registers.  Short sequences run one work-group per
//              (sequence, v-head).  Chunk operands are copied from global
//              memory straight into double-buffered LDS.
//   finish   : the state before each segment (S_{j+1} = S_j M_j + B_j), the
//              output correction O = O0 + OI S_j^T for segments >= 1, and the
//              final state of multi-segment sequences.
//
// Precision policy (fp32 accumulation everywhere): K, Q, V are bf16 inputs, so
// their products are exact.  S enters Q S^T as a single bf16 and K S^T as a
// single bf16, or as a bf16 hi + lo pair in chunks whose map bound shows slow
// decay (the state's rounding then survives many chunks); Tb and
// R = V - gam K S^T enter Delta = Tb R as fp16 (11 significant bits: one MFMA
// instead of three for a bf16 hi+lo pair), R scaled by a power of two into
// fp16's normal range first; the state update uses Delta' = tail Delta as a
// bf16 hi+lo pair; Aqk Delta (output only) is single bf16.  The fp32 state
// never leaves registers between chunks.
#include "gdn_common.h"
#include <algorithm>
#include <type_traits>
#include "../../include/gdn_mi355x.h"

namespace gdn {

constexpr int kChunk = 64;
constexpr int kFragTile = 512;               // one 16x32 MFMA operand fragment: 64 lanes x 8 16-bit values
// Gate block per (record, v-head): gam[64], tail[64], the chunk's map bound
// (below) at [128], the inverse of Tb's fp16 range scale (a power of two, 1
// for Tb in fp16's usual range; see prepass_heads) at [129], Gam[64] (log2 of
// the cumulative gate, from which the split consumer weights Aqk) at [192]
// (one 1 KB copy).
constexpr int kGamStride = 4 * kChunk;
constexpr int kBoundAt = 2 * kChunk;
constexpr int kTbScaleAt = kBoundAt + 1;
constexpr int kLgamAt = 3 * kChunk;
// The homogeneous part of one token's update multiplies the state by
// g_t (I - beta_t k_t k_t^T), whose 2-norm is at most g_t max(1, |1 - beta_t |k_t|^2|).
// The prepass stores the chunk's sum of log2 of these factors; once a run from
// the identity (an M-run) has accumulated less than kNegligibleLog2, its state
// and all later outputs are below 2^-30 (1e-9) of the state they multiply, far
// below the fp32 rounding of the results they are added to, and the run stops.
constexpr float kNegligibleLog2 = -30.0f;
// Chunks whose map bound is above this (log2) carry the state into X = K S^T
// as a bf16 hi + lo pair instead of one bf16 (see chain_chunk).
constexpr float kHiLoBoundLog2 = -8.0f;
constexpr int kMNegligible = 1 << 30;   // flag in the M-run table: the run stopped early, its map is negligible
constexpr int kFrags = 2;                    // per chunk in LDS: Tb (fp16), Aqk (bf16)

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

// Tb and Aqk are lower triangular, so fragments (m, d) = (0, 1) and (1, 1)
// (rows 0-31, columns 32-63) are zero.  Only the other six are stored, copied
// and multiplied: fragment (m, d) sits at slot frag_slot(m, d) of a matrix of
// kMatElems values.
__host__ __device__ constexpr bool frag_zero(int m, int d) { return m < 2 && d == 1; }
__host__ __device__ constexpr int frag_slot(int m, int d) { return m < 2 ? m : 2 * m - 2 + d; }
constexpr int kMatFrags = 6;
constexpr int kMatElems = kMatFrags * kFragTile;   // one packed 64x64 matrix
// ---- segments ---------------------------------------------------------------
// A long sequence is cut into segments of L chunks (L chosen per call by the
// planner).  Segment 0 runs from the true initial state.  Segment j >= 1 runs
// twice, concurrently with all others: the "B-run" from a zero state with the
// real V (outputs O0, final state B_j) and the "M-run" from the identity with
// V = 0 (outputs OI, final state M_j).  The recurrence is linear in (S, V), so
//   S_{j+1} = S_j M_j + B_j,          O_j = O0_j + OI_j S_j^T,
// which a short scan over segments and a parallel correction pass resolve.
constexpr int kMinSegChunks = 4;   // shortest M-run segment (the warm-up scheme may take 2 or 3)
constexpr int kMSlotElems = 8 * 4 * 2 * 64 * 8;   // M_j^T as bf16 hi / lo MFMA fragments, per head

// Upper bound on the segments of all multi-segment sequences: a sequence of
// tau tokens split into n >= 2 segments of L >= kMinSegChunks chunks has
// tau > 64 L and n = ceil(tau / 64 L) < 2 tau / 64 L, so n summed over
// sequences stays below T / (32 kMinSegChunks).
__host__ __device__ inline long long max_segments(long long tokens) {
  return tokens / (32 * kMinSegChunks) + 1;
}

// lists: header, multi-segment entries, later-segment table, runs (two int4
// each), short sequences.  Everything a kernel needs about one work item sits
// in one entry, so an item costs one dependent load before its data.
//   hdr[0] runs, [1] short sequences, [2] segment length L (chunks),
//   [3] multi-segment sequences, [4] segments >= 1 over all sequences,
//   [5] 1 when the batch uses warm-up segments (no M-runs, no finish work),
//   [8] split-consumer work queue (items claimed past each group's first),
//   [9] correction blocks appended by the consumer's M-runs
//   multi[e]   = (seq, first slot, segments, 0)
//   segs[i]    = (first token lo, hi, tokens in the segment | j << 17, slot of
//                 segment j - 1) for every segment j >= 1 (L <= 1024 chunks:
//                 at most 65536 tokens)
//   runs[2i]   = (seq, flags | tokens of the run's last chunk << 8 | segment
//                 j << 16, final-state slot or -1 for new_state, first record)
//   runs[2i+1] = (first token lo, hi, chunks with records, chunks)
//   flags: kRunM (M-run), kRunFromState (initial state from `state`),
//          kRunWarm (warm-up run, below); final-state slot -1: new_state,
//          -2: none (a warm-up run of a segment before the last)
//   shorts[i]  = (seq, record of its chunk or -1 when it has none, first token
//                 lo, first token hi | tokens << 16) for sequences of at most
//                 one chunk
constexpr int kListHdr = 16;
constexpr int kRunM = 1;
constexpr int kRunFromState = 2;
constexpr int kRunWarm = 4;
// Warm-up segments.  When every v-head's segment map becomes negligible within
// a few chunks, segment j >= 1 needs no M-run and no correction: its run starts
// W chunks before the segment, from a zero state, with W the fewest preceding
// chunks whose map bounds sum below kNegligibleLog2.  The state it carries
// into the segment then differs from the true one by less than 2^-30 of the
// state those chunks started from (the criterion an M-run stops on), and it
// discards the outputs of the warm-up chunks.  The run finds W itself from the
// prepass's chunk bounds; if they never get that low it starts at the
// sequence's first chunk from the true initial state, which is exact.  The
// planner takes this scheme when its estimate of every head's warm-up (from
// A_log and dt_bias) is at most kWarmMaxChunks.
constexpr int kWarmMaxChunks = 4;
constexpr int kSlotNone = -2;

// Finish work: a correction block is one or more chunks of one (segment,
// v-head); wave w of a finish group corrects 16-token tile w of each chunk.
// A block first forms the segment's starting state, which for segment j can
// take up to j - 1 scan steps.  The M-run of a segment j >= kFinBlockSeg that
// formed more than kFinBlockChunks chunks lists blocks of kFinBlockChunks
// chunks, so that state is formed once per block rather than once per chunk;
// otherwise it lists one block per chunk, and the blocks run in parallel.
constexpr int kFinThreads = 256;
constexpr int kFinGroups = 512;   // one round at two groups per CU (the launch bounds)
static_assert(kFinGroups == 64 * 8, "finish item permutation: 64 items per XCD");
constexpr int kFinBlockChunks = 4;
constexpr int kFinBlockSeg = 3;
static_assert(kFinThreads / 64 == kChunk / 16, "finish tiling: one wave per 16-token tile");
__host__ __device__ inline long long max_runs(int num_seqs, long long gcap) { return 2 * gcap + num_seqs; }

struct ListView {
  int* hdr;
  int4* multi;
  int4* segs;
  int4* runs;
  int4* shorts;
};

__host__ __device__ inline ListView list_view(int* lists, int num_seqs, long long gcap) {
  ListView v;
  v.hdr = lists;
  v.multi = reinterpret_cast<int4*>(lists + kListHdr);
  v.segs = v.multi + num_seqs;
  v.runs = v.segs + gcap;
  v.shorts = v.runs + 2 * max_runs(num_seqs, gcap);
  return v;
}

__host__ __device__ inline size_t list_ints(int num_seqs, long long gcap) {
  return kListHdr + 4 * static_cast<size_t>(num_seqs) + 4 * static_cast<size_t>(gcap) +
         8 * static_cast<size_t>(max_runs(num_seqs, gcap)) + 4 * static_cast<size_t>(num_seqs);
}

// ---- workspace layout -------------------------------------------------------
struct WsLayout {
  size_t frag_off;     // u16  [R][8][kMatElems] Tb (fp16)
  size_t gam_off;      // f32  [R][8][kGamStride] (gam, tail, map bound, Gam)
  size_t start_off;    // i32  [N + 1]           record start per sequence
  size_t list_off;     // i32  lists (see list_view)
  size_t rec_off;      // i32x4[R]               (seq, first token, length, 0)
  size_t slotb_off;    // f32  [G][8][128][128]  S_1 (slot of segment 0), B_j (slots of segments j >= 1)
  size_t slotm_off;    // u16  [G][8][kMSlotElems] M_j^T fragments
  size_t oi_off;       // u16  [T][8][128]       M-run outputs OI (rows of segments >= 1)
  size_t mval_off;     // i32  [G][8]            M-run chunks whose outputs OI were formed | kMNegligible
  size_t fix_off;      // i32x4[8 R][2]          correction blocks (segs entry; v-head, first, last chunk)
  size_t total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline long long max_records(int num_seqs, long long tokens) {
  return (tokens + kChunk - 1) / kChunk + num_seqs;
}

// Layout for gcap segment slots (0 .. max_segments(tokens)): the planner only
// picks segment lengths whose slots fit, so any gcap gives the same results;
// with none, no sequence is segmented and the M-run outputs need no storage.
__host__ __device__ inline WsLayout ws_layout(int num_seqs, long long tokens, long long gcap) {
  WsLayout L;
  const size_t R = static_cast<size_t>(max_records(num_seqs, tokens));
  const size_t G = static_cast<size_t>(gcap);
  const size_t N = static_cast<size_t>(num_seqs);
  size_t off = 0;
  L.frag_off = off;  off = align256(off + R * kVHeads * kMatElems * sizeof(uint16_t));
  L.gam_off = off;   off = align256(off + R * kVHeads * kGamStride * sizeof(float));
  L.start_off = off; off = align256(off + (N + 1) * sizeof(int));
  L.list_off = off;  off = align256(off + list_ints(num_seqs, static_cast<long long>(G)) * sizeof(int));
  L.rec_off = off;   off = align256(off + R * sizeof(int4));
  L.slotb_off = off; off = align256(off + G * kVHeads * kHeadState * sizeof(float));
  L.slotm_off = off; off = align256(off + G * kVHeads * kMSlotElems * sizeof(uint16_t));
  L.oi_off = off;    off = align256(off + (G > 0 ? static_cast<size_t>(tokens) : 0) * kVHeads * kDim * sizeof(uint16_t));
  L.mval_off = off;  off = align256(off + G * kVHeads * sizeof(int));
  // a block covers formed chunks of one M-run, whose records are its own: at most 8 R blocks
  L.fix_off = off;   off = align256(off + R * kVHeads * 2 * sizeof(int4));
  L.total = off;
  return L;
}

// Segment slots of the default workspace: each costs 1 MiB (a state and a
// segment map per v-head).  The planner's best segmentings of the benchmark
// batches use at most a few dozen (16 sequences of 16384 tokens: 10).
constexpr long long kDefaultSlots = 48;

// The most slots (up to what the batch can use) whose layout fits `bytes`, or
// -1 when not even the layout without slots fits.
inline long long slots_fitting(int num_seqs, long long tokens, size_t bytes) {
  long long lo = 0, hi = max_segments(tokens);
  if (ws_layout(num_seqs, tokens, 0).total > bytes) return -1;
  while (lo < hi) {   // the layout grows with gcap
    const long long mid = lo + (hi - lo + 1) / 2;
    if (ws_layout(num_seqs, tokens, mid).total <= bytes) lo = mid; else hi = mid - 1;
  }
  return lo;
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
// plan: record numbering, segment length, consumer work lists
// ============================================================================
constexpr int kPlanThreads = 1024;
constexpr int kConsumerGroups = 256;     // persistent work-groups per consumer kind (one per CU)

// Sequences of at least this many chunks run on the split consumer (chunk
// time bounds the call); shorter ones on the full-head consumer (throughput).
constexpr int kLongChunks = 2;

// ---- wave / work-group reductions on DPP (no LDS traffic inside a wave) ----
// update_dpp with old = 0 and bound_ctrl off: lanes whose source lies outside
// their row (or rows masked off) read 0.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ int dpp0(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xf, false);
}

// Inclusive prefix sum over the 64 lanes: row_shr 1, 2, 4, 8 within rows of
// 16, then row_bcast 15 / 31 carry the row totals into the rows above.
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += dpp0<0x111>(x);
  x += dpp0<0x112>(x);
  x += dpp0<0x114>(x);
  x += dpp0<0x118>(x);
  x += dpp0<0x142, 0xa>(x);
  x += dpp0<0x143, 0xc>(x);
  return x;
}

__device__ __forceinline__ int wave_sum(int x) { return __builtin_amdgcn_readlane(wave_incl_sum(x), 63); }

// Sum over the 64 lanes (fp32, every lane gets it): DPP within rows of 16, then
// the four row totals.
template <int CTRL>
__device__ __forceinline__ float dppf0(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float dppf0r(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWS, 0xf, false));
}

// Inclusive prefix sum over the 64 lanes (fp32), as wave_incl_sum.
__device__ __forceinline__ float wave_incl_sumf(float x) {
  x += dppf0<0x111>(x);
  x += dppf0<0x112>(x);
  x += dppf0<0x114>(x);
  x += dppf0<0x118>(x);
  x += dppf0r<0x142, 0xa>(x);
  x += dppf0r<0x143, 0xc>(x);
  return x;
}

__device__ __forceinline__ float wave_sumf(float x) {
  x += dppf0<0x111>(x);
  x += dppf0<0x112>(x);
  x += dppf0<0x114>(x);
  x += dppf0<0x118>(x);
  auto lane_f = [&](int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
  return (lane_f(15) + lane_f(31)) + (lane_f(47) + lane_f(63));
}

// Maximum over the lanes of non-negative values (0 is the identity).
__device__ __forceinline__ int wave_max0(int x) {
  x = max(x, dpp0<0x111>(x));
  x = max(x, dpp0<0x112>(x));
  x = max(x, dpp0<0x114>(x));
  x = max(x, dpp0<0x118>(x));
  x = max(x, dpp0<0x142, 0xa>(x));
  x = max(x, dpp0<0x143, 0xc>(x));
  return __builtin_amdgcn_readlane(x, 63);
}

// Power-of-two scale for an fp16 operand (one value per wave), from each
// lane's maximum |x|: 1 while every |x| of the wave is below 2^15 and at
// least one reaches 2^-4 (checked with two ballots, no cross-lane reduction);
// otherwise the wave maximum goes to [2^10, 2^11), so the operand keeps fp16's
// 11 significant bits at any magnitude.  Zero, inf and NaN maxima keep scale 1
// (they pass through as in fp32).  Used for R = V - gam X (the caller divides
// Delta = Tb R by the same power of two) and for Tb in the prepass.
__device__ __forceinline__ float fp16_range_scale(float mx) {
  const bool big = __builtin_amdgcn_ballot_w64(mx >= 32768.0f) != 0;
  const bool small = __builtin_amdgcn_ballot_w64(mx >= 0.0625f) == 0;
  if (!big && !small) return 1.0f;
  const int bits = wave_max0(__float_as_int(mx));   // non-negative floats order as integers
  if (bits == 0 || bits >= 0x7f800000) return 1.0f;
  const int e = max((bits >> 23) - 127, -117);      // floor(log2 max), subnormals clamped
  return __int_as_float((137 - e) << 23);           // 2^(10 - e)
}

// Inclusive prefix sum over the NT threads of the work-group (wave_tot: NT / 64 ints).
template <int NT>
__device__ __forceinline__ int block_scan(int x, int* wave_tot) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  x = wave_incl_sum(x);
  if (lane == 63) wave_tot[wv] = x;
  __syncthreads();
  int add = 0;
  for (int j = 0; j < wv; ++j) add += wave_tot[j];
  __syncthreads();
  return x + add;
}

// K prefix sums at once: x becomes the inclusive scan, total the block sums
// (wave_tot: NT / 64 * K ints).
template <int NT, int K>
__device__ __forceinline__ void block_scan_v(int (&x)[K], int* wave_tot, int (&total)[K]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < K; ++i) x[i] = wave_incl_sum(x[i]);
  if (lane == 63) {
#pragma unroll
    for (int i = 0; i < K; ++i) wave_tot[wv * K + i] = x[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < K; ++i) {
    int add = 0, tot = 0;
    for (int j = 0; j < NT / 64; ++j) {
      const int t = wave_tot[j * K + i];
      add += j < wv ? t : 0;
      tot += t;
    }
    x[i] += add;
    total[i] = tot;
  }
  __syncthreads();
}

// Candidate segment lengths (chunks): 2, 3 (warm-up batches only), 4, 6, ...,
// 32, then 40, 48, 64, 80, 96, 128, ... (5, 6, 8 x 2^k) up to 1024, and "no
// split", in increasing order.
constexpr int kSegCands = 33;
constexpr int kShortCands = 2;   // the candidates below kMinSegChunks
__device__ __forceinline__ int seg_cand(int i) {
  if (i >= kSegCands - 1) return 1 << 30;
  if (i < kShortCands) return 2 + i;
  i -= kShortCands;
  if (i < 15) return 4 + 2 * i;
  const int j = i - 15, m = j % 3;
  return (m == 0 ? 5 : (m == 1 ? 6 : 8)) << (3 + j / 3);
}

// Partial runs are ordered by length, longest first: exact below 64 chunks,
// by power of two above.
constexpr int kBuckets = 96;
__device__ __forceinline__ int len_bucket(int len) { return len < 64 ? len : 64 + (31 - __clz(len)); }

// Runs of one sequence for segment length L.  Segments 0 .. nseg-2 have L
// chunks, the last one `last` (1 .. L).  Full-length runs: segment 0's, and
// the B- and M-run of every other full segment; a shorter last segment gives
// one or two "partial" runs.
struct SeqPlan {
  int is_long, nseg, multi, full_seg, full_runs, part_runs, last;
};

__device__ __forceinline__ SeqPlan seq_plan(int nch, int L, bool warm) {
  SeqPlan p = {0, 0, 0, 0, 0, 0, 0};
  if (nch < kLongChunks) return p;
  p.is_long = 1;
  p.nseg = (nch - 1) / L + 1;
  p.last = nch - (p.nseg - 1) * L;
  p.full_seg = p.last == L ? p.nseg : p.nseg - 1;
  if (warm) {   // one run per segment, no M-runs, nothing for the finish
    p.multi = 0;
    p.full_runs = p.full_seg;
    p.part_runs = p.last == L ? 0 : 1;
  } else {
    p.multi = p.nseg >= 2 ? 1 : 0;
    p.full_runs = p.full_seg > 0 ? 2 * p.full_seg - 1 : 0;
    p.part_runs = p.last == L ? 0 : (p.nseg == 1 ? 1 : 2);
  }
  return p;
}

// Scratch ints used by plan_batch.
constexpr int kPsVals = 3 * kSegCands + 3;
constexpr int kPsCand = 0;                                   // [waves][kPsVals]
constexpr int kPsScan = kPsCand + (kPlanThreads / 64) * kPsVals;   // [waves][5]
constexpr int kPsHist = kPsScan + (kPlanThreads / 64) * 5;
constexpr int kPsCur = kPsHist + kBuckets;
constexpr int kPsMisc = kPsCur + kBuckets;
constexpr int kPlanScratch = kPsMisc + 4;

// Plans the call for the whole batch with one work-group of NT threads, thread
// i owning a contiguous range of sequences: rec_start (chunk record of each
// sequence's first chunk), the segment length, and the work lists of the
// split consumer (runs, longest first), the full-head consumer (short
// sequences), the scan (multi-segment sequences) and the correction (segments
// >= 1).
//
// Segment length: for each candidate L an estimate of the split consumer's
// critical path in chunk steps, the smallest winning (ties to the longer L).
// With M-runs: max(L + o, (16 W(L) + 16 o runs(L)) / groups), W(L) = sum over
// long sequences of (2 nch - min(nch, L)) chunk runs per (value half, v-head),
// o the per-item overhead, plus about half a step per segment for the scan and
// 1.5 for segmenting at all (and a scan term for slowly decaying heads).  With
// warm-up runs: the runs' list schedule on groups / 16 machines (longest run
// or balanced load plus a last-round tail; see the evaluation below).
// Candidates whose segments would not fit the workspace slots are skipped.
// Returns the thread's first record index.  t0_first / t1_first: bounds of the
// thread's first sequence when the caller already read them (t1_first < 0:
// not known).
template <int NT>
__device__ int plan_batch(const void* __restrict__ cu, int is64, int num_seqs, long long T, int R, int gcap,
                          const float* __restrict__ A_log, const float* __restrict__ dt_bias,
                          int* __restrict__ rec_start, int* __restrict__ lists, int* ps, int& total_recs,
                          long long t0_first = 0, long long t1_first = -1) {
  constexpr int kW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int per = (num_seqs + NT - 1) / NT;
  const int s_begin = min(tid * per, num_seqs);
  const int s_end = min(num_seqs, s_begin + per);
  long long b0 = 0, b1 = 0;   // bounds of the first sequence, read once
  if (s_begin < s_end) {
    if (t1_first >= 0) {
      b0 = t0_first;
      b1 = t1_first;
    } else {
      seq_bounds(cu, is64, s_begin, T, b0, b1);
    }
  }
  auto bounds = [&](int s, long long& t0, long long& t1) {
    if (s == s_begin) {
      t0 = b0;
      t1 = b1;
    } else {
      seq_bounds(cu, is64, s, T, t0, t1);
    }
  };
  auto chunks = [&](int s) {
    long long t0, t1;
    bounds(s, t0, t1);
    return static_cast<int>((t1 - t0 + kChunk - 1) / kChunk);
  };

  // ---- pass 1: statistics per candidate segment length ----
  // A: sum of min(nch, L); B: slots (segments of multi-segment sequences);
  // C: runs (2 nseg - 1 per long sequence)
  int A[kSegCands], B[kSegCands], C[kSegCands];
#pragma unroll
  for (int i = 0; i < kSegCands; ++i) A[i] = B[i] = C[i] = 0;
  int suml = 0, maxl = 0, nlong = 0;
  for (int s = s_begin; s < s_end; ++s) {
    const int nch = chunks(s);
    if (nch < kLongChunks) continue;
    suml += nch;
    maxl = max(maxl, nch);
    ++nlong;
#pragma unroll
    for (int i = 0; i < kSegCands; ++i) {
      const int Lc = seg_cand(i);
      const int nseg = (nch - 1) / Lc + 1;
      A[i] += min(nch, Lc);
      B[i] += nseg > 1 ? nseg : 0;
      C[i] += 2 * nseg - 1;
    }
  }
  // waves without long sequences (most of a short-sequence batch) skip the reductions
  if (__builtin_amdgcn_ballot_w64(maxl > 0) != 0) {
#pragma unroll
    for (int i = 0; i < kSegCands; ++i) {
      A[i] = wave_sum(A[i]);
      B[i] = wave_sum(B[i]);
      C[i] = wave_sum(C[i]);
    }
    suml = wave_sum(suml);
    maxl = wave_max0(maxl);
    nlong = wave_sum(nlong);
  }
  if (lane == 0) {
    int* pw = ps + kPsCand + wv * kPsVals;
#pragma unroll
    for (int i = 0; i < kSegCands; ++i) {
      pw[i] = A[i];
      pw[kSegCands + i] = B[i];
      pw[2 * kSegCands + i] = C[i];
    }
    pw[3 * kSegCands] = suml;
    pw[3 * kSegCands + 1] = maxl;
    pw[3 * kSegCands + 2] = nlong;
  }
  for (int i = tid; i < 2 * kBuckets; i += NT) ps[kPsHist + i] = 0;
  __syncthreads();
  if (wv == 0) {
    // per v-head (lanes 0-7) the log2 bound of one chunk's map, estimated from
    // the per-head constants (a = 0): 64 log2 g = -64 log2(e) exp(A_log) softplus(dt_bias)
    const float hb = lane < kVHeads
                         ? kChunk * kLog2e * log_decay(A_log[min(lane, kVHeads - 1)], 0.0f,
                                                       dt_bias[min(lane, kVHeads - 1)])
                         : -1.0e30f;
    // fraction of v-heads that decay slowly (see below)
    const bool slow_h = lane < kVHeads && 2.0f * hb > kNegligibleLog2;
    const float slow_frac = static_cast<float>(__popcll(__builtin_amdgcn_ballot_w64(slow_h))) / kVHeads;
    // warm-up chunks each head needs (estimate), and the scheme
    const int wh = hb < kNegligibleLog2 ? 1 : (hb < 0.f ? static_cast<int>(ceilf(kNegligibleLog2 / hb)) : 1 << 20);
    const int w_est = wave_max0(min(wh, 1 << 20));
    const bool warm = w_est <= kWarmMaxChunks;
    // lane i < kSegCands evaluates candidate i, in chunk steps of the split
    // consumer: the longest run and the average work-group load (chunk runs
    // plus a per-item overhead) bound the critical path; the scan adds half a
    // step per segment and segmenting at all 1.5 steps.  The minimum over the
    // lanes wins, ties to the longer segments.
    float sl = 0.f, a = 0.f, runs = 0.f, nl = 0.f;
    long long slots = 0;
    int ml = 0;
    const int ci = min(lane, kSegCands - 1);
    for (int j = 0; j < kW; ++j) {
      const int* pj = ps + kPsCand + j * kPsVals;
      sl += static_cast<float>(pj[3 * kSegCands]);
      ml = max(ml, pj[3 * kSegCands + 1]);
      nl += static_cast<float>(pj[3 * kSegCands + 2]);
      a += static_cast<float>(pj[ci]);
      slots += pj[kSegCands + ci];
      runs += static_cast<float>(pj[2 * kSegCands + ci]);
    }
    constexpr float kItemOverhead = 1.0f;   // chunk steps per work item (metadata, state, first copies)
    const int Lc = seg_cand(ci);
    const int nseg_max = ml > 0 ? (ml - 1) / Lc + 1 : 0;
    float est;
    if (warm) {
      // Warm-up scheme: one run per segment (T of them), each later segment
      // W chunks longer; the work-groups take a run's 16 items together, so
      // the packing is that of T runs on kConsumerGroups / 16 machines:
      // the longest run, or the balanced load plus a quarter of an average
      // run for the last round when there is more than one.  Item overhead
      // (descriptor, warm-up bounds, first copies, final stores) about 1.5
      // chunk steps.  Fitted with a list-scheduling model of the consumer
      // against its measured step and item costs (c3: L = 18, 2 x 8192
      // tokens: 16, 4 x 16384: 64, all measured faster than the earlier
      // estimate's 20, 28 and 96).
      constexpr float kWarmItem = 1.5f, kTailShare = 0.25f, kSegmented = 0.75f;
      constexpr float kMachines = static_cast<float>(kConsumerGroups / 16);
      const float T = 0.5f * (runs + nl);                      // runs = sum of 2 nseg - 1
      const float work = sl + static_cast<float>(w_est) * (T - nl);
      const float longest = ml > Lc ? static_cast<float>(Lc + w_est) : static_cast<float>(ml);
      const float balanced = (work + kWarmItem * T) / kMachines;
      const float tail = T > kMachines ? kTailShare * (work / fmaxf(T, 1.f) + kWarmItem) : 0.f;
      est = fmaxf(longest + kWarmItem, balanced + tail) + (nseg_max > 1 ? kSegmented : 0.f);
    } else {
      // M-run scheme: W(L) counts the M-runs of later segments.  The scan
      // adds about half a step per segment and segmenting at all 1.5 steps.
      const float per_wg = (16.f * (2.f * sl - a) + kItemOverhead * 16.f * runs) / kConsumerGroups;
      const float crit = static_cast<float>(min(Lc, ml)) + kItemOverhead;
      est = fmaxf(crit, per_wg) + (nseg_max > 1 ? 0.5f * static_cast<float>(nseg_max - 1) + 1.5f : 0.f);
    }
    // Slowly decaying heads: their segment maps never become negligible, so
    // every correction block of segment j >= 2 in the finish first takes j - 1
    // scan steps.  The heads' chunk map bound is estimated from the per-head
    // constants (a = 0): 64 log2 g = -64 log2(e) exp(A_log) softplus(dt_bias);
    // a head is slow when two chunks do not reach the negligible bound.  Such
    // batches pay about kScanStepCost chunk steps per chunk of the longest
    // sequence's segments j >= 2, weighted by j - 1 (measured with forced
    // segment lengths on configuration 3 with near-1 decay).
    if (!warm && slow_frac > 0.f && nseg_max >= 3) {
      constexpr float kScanStepCost = 0.45f;
      const int last = ml - (nseg_max - 1) * Lc;
      const float pj = static_cast<float>(Lc) * static_cast<float>((nseg_max - 3) * (nseg_max - 2) / 2) +
                       static_cast<float>(last) * static_cast<float>(nseg_max - 2);
      est += slow_frac * kScanStepCost * pj;
    }
    // key: estimate in 1/16 steps, then the longer candidate; invalid lanes hold
    // the maximum.  No slot is written in the warm-up scheme, but the slot
    // bound still applies: the run table holds max_runs(N, gcap) = N + 2 gcap
    // runs, and with at most gcap later segments the runs (one per segment)
    // stay within it.
    const int q = static_cast<int>(fminf(est * 16.f, 1.0e7f));
    // segments below kMinSegChunks only without M-runs (the workspace's slots
    // are sized for M-run segments of at least kMinSegChunks)
    const bool allowed = lane < kSegCands && slots <= gcap && (warm || Lc >= kMinSegChunks);
    const int key = allowed ? q * 64 + (63 - lane) : 0x7fffffff;
    // minimum over the lanes: the maximum of the complements
    const int best = 0x7fffffff - wave_max0(0x7fffffff - key);
    if (lane == 0) {
      ps[kPsMisc] = seg_cand(63 - (best & 63));
      ps[kPsMisc + 1] = warm ? 1 : 0;
    }
  }
  __syncthreads();
  const int L = ps[kPsMisc];
  const bool warm = ps[kPsMisc + 1] != 0;

  // ---- pass 2: per-sequence counts and their prefix sums ----
  // v: records, short sequences, multi-segment sequences, slots, full runs
  int v[5] = {0, 0, 0, 0, 0};
  for (int s = s_begin; s < s_end; ++s) {
    const int nch = chunks(s);
    const SeqPlan p = seq_plan(nch, L, warm);
    v[0] += nch;
    v[1] += p.is_long ? 0 : 1;
    v[2] += p.multi;
    v[3] += p.multi ? p.nseg : 0;
    v[4] += p.full_runs;
    if (p.part_runs) atomicAdd(&ps[kPsHist + len_bucket(p.last)], p.part_runs);
  }
  int own[5], tot[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) own[i] = v[i];
  block_scan_v<NT, 5>(v, ps + kPsScan, tot);
  total_recs = tot[0];
  const ListView lv = list_view(lists, num_seqs, gcap);
  if (wv == 0) {
    // partial runs follow the full-length ones, longest first: descending
    // exclusive prefix of the bucket counts, two buckets per lane
    const int b0_ = kBuckets - 1 - 2 * lane, b1_ = b0_ - 1;
    const int h0 = lane < kBuckets / 2 ? ps[kPsHist + b0_] : 0;
    const int h1 = lane < kBuckets / 2 ? ps[kPsHist + b1_] : 0;
    const int inc = wave_incl_sum(h0 + h1);
    const int ex = tot[4] + inc - h0 - h1;
    if (lane < kBuckets / 2) {
      ps[kPsCur + b0_] = ex;
      ps[kPsCur + b1_] = ex + h0;
    }
    if (lane == 0) {
      lv.hdr[8] = 0;   // work queue
      lv.hdr[9] = 0;   // correction blocks
    }
    if (lane == 63) {
      lv.hdr[0] = tot[4] + inc;
      lv.hdr[1] = tot[1];
      lv.hdr[2] = L;
      lv.hdr[3] = tot[2];
      lv.hdr[4] = tot[3] - tot[2];
      lv.hdr[5] = warm ? 1 : 0;
      rec_start[num_seqs] = min(tot[0], R);
    }
  }
  __syncthreads();

  // ---- pass 3: emit ----
  int rb = v[0] - own[0], sp = v[1] - own[1], mp = v[2] - own[2];
  int gb = v[3] - own[3], fp = v[4] - own[4];
  const int rb0 = rb;
  for (int s = s_begin; s < s_end; ++s) {
    long long t0, t1;
    bounds(s, t0, t1);
    const int nch = static_cast<int>((t1 - t0 + kChunk - 1) / kChunk);
    const SeqPlan p = seq_plan(nch, L, warm);
    const int rec0 = rb;
    rec_start[s] = rb;
    rb += nch;
    if (!p.is_long) {
      // chunks whose records exist (overlapping cu_seqlens can exhaust the capacity)
      const int rec = nch > 0 && rec0 < R ? rec0 : -1;
      lv.shorts[sp++] = make_int4(s, rec, static_cast<int>(t0 & 0xffffffffLL),
                                  static_cast<int>(t0 >> 32) | (static_cast<int>(t1 - t0) << 16));
      continue;
    }
    const int g0 = p.multi ? gb : 0;
    if (p.multi) {
      // later-segment table: entries gb - mp .. (one per segment >= 1)
      lv.multi[mp] = make_int4(s, gb, p.nseg, 0);
      for (int j = 1; j < p.nseg; ++j) {
        const long long c0 = t0 + static_cast<long long>(j) * L * kChunk;
        const int tok = static_cast<int>(min(t1 - c0, static_cast<long long>(L) * kChunk));
        lv.segs[gb - mp + j - 1] = make_int4(static_cast<int>(c0 & 0xffffffffLL), static_cast<int>(c0 >> 32),
                                             tok | (j << 17), gb + j - 1);
      }
      ++mp;
      gb += p.nseg;
    }
    // one run of segment j (flags: kRunM / kRunFromState) at list position pos
    auto emit_run = [&](int pos, int j, bool mrun) {
      const long long i0 = static_cast<long long>(j) * L;
      const int nrun = static_cast<int>(min(static_cast<long long>(nch) - i0, static_cast<long long>(L)));
      const long long c0 = t0 + i0 * kChunk;
      // tokens of the run's last chunk: 64 unless the run ends the sequence
      const long long run_end = min(t1, c0 + static_cast<long long>(nrun) * kChunk);
      const int last_tok = static_cast<int>(run_end - (c0 + static_cast<long long>(nrun - 1) * kChunk));
      const long long rfirst = rec0 + i0;
      // chunks whose records exist (overlapping cu_seqlens can exhaust the capacity)
      const int nvalid = static_cast<int>(max(0LL, min(static_cast<long long>(nrun), R - rfirst)));
      const int flags = (mrun ? kRunM : 0) | (!mrun && j == 0 ? kRunFromState : 0) | (warm && j > 0 ? kRunWarm : 0);
      const int slot = p.multi ? g0 + j : (warm && j < p.nseg - 1 ? kSlotNone : -1);
      lv.runs[2 * pos] = make_int4(s, flags | (last_tok << 8) | (j << 16), slot,
                                   static_cast<int>(min(rfirst, 0x7fffffffLL)));
      lv.runs[2 * pos + 1] = make_int4(static_cast<int>(c0 & 0xffffffffLL), static_cast<int>(c0 >> 32), nvalid, nrun);
    };
    for (int j = 0; j < p.full_seg; ++j) {
      emit_run(fp++, j, false);
      if (j > 0 && !warm) emit_run(fp++, j, true);
    }
    if (p.part_runs) {
      const int pos = atomicAdd(&ps[kPsCur + len_bucket(p.last)], p.part_runs);
      const int j = p.nseg - 1;
      emit_run(pos, j, false);
      if (p.part_runs == 2) emit_run(pos + 1, j, true);
    }
  }
  return rb0;
}

// Separate planning launch for large batches: plan_batch plus the flat record
// table the prepass reads.
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(
    const void* __restrict__ cu, int is64, int num_seqs, long long T, int R, int gcap,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    int* __restrict__ rec_start, int4* __restrict__ recs, int* __restrict__ lists) {
  __shared__ int ps[kPlanScratch];
  const int tid = threadIdx.x;
  const int per = (num_seqs + kPlanThreads - 1) / kPlanThreads;
  const int s_begin = min(tid * per, num_seqs);
  const int s_end = min(num_seqs, s_begin + per);
  int total_recs;
  int base = plan_batch<kPlanThreads>(cu, is64, num_seqs, T, R, gcap, A_log, dt_bias, rec_start, lists, ps,
                                      total_recs);
  for (int s = s_begin; s < s_end; ++s) {
    long long t0, t1;
    seq_bounds(cu, is64, s, T, t0, t1);
    // overlapping (non-monotonic) cu_seqlens can ask for more than R records:
    // records past the capacity are dropped and the consumer skips them
    for (long long c0 = t0; c0 < t1; c0 += kChunk, ++base) {
      const int len = static_cast<int>(min(static_cast<long long>(kChunk), t1 - c0));
      if (base < R) recs[base] = make_int4(s, static_cast<int>(c0), len, 0);
    }
  }
  const int total = min(total_recs, R);
  for (int r = total + tid; r < R; r += kPlanThreads) recs[r] = make_int4(-1, 0, 0, 0);
}

// ============================================================================
// device helpers shared by the prepass and the consumer
// ============================================================================
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16h(const f16x8& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// K / Q rows in LDS keep natural column order; the 16-byte chunk j of row t is
// stored at position j ^ kq_swz(t).  kq_swz is linear over GF(2) in t & 15:
// bits 0-1 of t move to bits 2-3, bit 2 adds 2 and bit 3 adds 3.  Chosen by
// measurement on gfx950 (64 banks) among all linear maps: the row reads (8
// consecutive k of 16 rows, ds_read_b128) run conflict-free and the transposed
// reads (4 consecutive k of 4 rows x 4 chunks, ds_read_b64_tr_b16) at their
// floor of two passes per 32 lanes; the earlier map
// ((t & 3) << 2) | ((t >> 2) & 3) took twice as long for the row reads.
__device__ __forceinline__ int kq_swz(int t) {
  return ((t & 3) << 2) | ((((t >> 2) & 1) << 1) ^ (((t >> 3) & 1) * 3));
}

// 16 bytes per lane from global memory straight into LDS: lane i of the wave
// writes bytes [16 i, 16 i + 16) after the wave-uniform LDS address.  AUX is
// the cache policy: 2 (nt) streams data that is read exactly once.
template <int AUX = 0>
__device__ __forceinline__ void dma16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, AUX);
}

typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// gfx950 transposed LDS read: in each 16-lane group, lane i receives element
// (i & 3) of the 8-byte vectors addressed by lanes i/4, i/4+4, i/4+8, i/4+12.
__device__ __forceinline__ u32x2 lds_tr16(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// Work-group barrier that waits for this wave's LDS operations only; its
// global-to-LDS copies stay in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0), vmcnt / expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ============================================================================
// prepass: chunk-local WY terms, one wave per item
// ============================================================================
// Each wave runs whole items on its own, with no work-group barrier: the K / Q
// rows come straight from global memory into MFMA operand registers (16 bytes
// of a row per lane is both the A and the B fragment of a gram), the gates sit
// on the lanes (lane = token), and only the 16x16 diagonal blocks of the
// triangular inverse pass through LDS.  An item is one (record, v-head) when
// the batch has at most 3072 of them (each v-head's phases on its own wave:
// the shortest latency; two waves per SIMD up to 2048 items, three beyond),
// else one (record, q/k head) whose wave loads the rows and forms the gram
// once and runs both v-heads of the GVA pair (two waves per SIMD: up to 512
// records at once).
//
// The inverse is formed transposed: with U = I + N^T (unit upper) and
// W = U^{-1} = T^T, the 16x16 blocks satisfy
//   W_aa = (T_aa)^T,   W_ab = -W_aa sum_{m=a+1..b} U_am W_mb   (a < b),
// T_aa by forward substitution (one lane per column), the off-diagonal blocks
// on MFMA.  W in MFMA C layout holds Tb^T = diag(beta) W with lane = row of
// Tb, which is exactly the register order of Tb's A fragments.
constexpr int kPrepassThreads = 256;              // four independent waves
constexpr int kPrepassWaves = kPrepassThreads / 64;
constexpr int kPrepassMaxGroups = 512;             // two per CU: eight waves, two per SIMD

struct __align__(16) PrepassWaveSmem {   // per v-head of the item
  float lgam[kGva][kChunk];    // Gam_t / ln 2 (inclusive scan of log2 g)
  float beta[kGva][kChunk];
  // diagonal blocks N_aa, column-major (nt[a][column][row]); the forward
  // substitution then overwrites each with its inverse T_aa (a wave reads all of
  // its N columns before its first T store)
  float nt[kGva][4][16][16];
};

// Batches of at most kFusedPlanSeqs sequences number their records inside the
// prepass (no plan launch): wave 0 of each work-group scans the chunk counts
// of all sequences once into LDS, and each item finds its sequence there with
// a ballot.
constexpr int kFusedPlanSeqs = 512;
constexpr int kFusedBlocks = kFusedPlanSeqs / 64;

struct PrepassSeqSmem {
  int incl[kFusedPlanSeqs];          // inclusive prefix of the chunk counts (past the last: the total)
  long long s0[kFusedPlanSeqs];      // sequence bounds (clamped)
  long long s1[kFusedPlanSeqs];
};

struct PrepassSmem {
  union {
    PrepassWaveSmem w[kPrepassWaves];
    int plan[kPlanScratch];      // planner scratch (work-group 0 of a fused launch)
  } u;
  PrepassSeqSmem seq;
};


// acc + X Y for 16x16 fp32 blocks with X^T and Y in C layout (lane (lg, l16),
// register r: row 4 lg + r, column l16), on two bf16 MFMAs with both operands
// split into bf16 hi + lo: X_hi Y_hi + X_lo Y_hi + X_hi Y_lo (relative error
// about 2^-16, far below the fp16 rounding of Tb).  Depth slot s of lane group
// lg is product depth 4 lg + (s & 3): the A operand holds X_hi in slots 0-3
// and X_lo in slots 4-7; the first B operand holds Y_hi in both halves, the
// second Y_lo in slots 0-3 and zeros in 4-7.  An operand used in several
// products is split once.
__device__ __forceinline__ bf16x8 split_x(const f32x4& xt) {
  const uint32_t xh0 = pack_bf2(xt[0], xt[1]), xh1 = pack_bf2(xt[2], xt[3]);
  const uint32_t xl0 = pack_bf2(xt[0] - bf_lo(xh0), xt[1] - bf_hi(xh0));
  const uint32_t xl1 = pack_bf2(xt[2] - bf_lo(xh1), xt[3] - bf_hi(xh1));
  return __builtin_bit_cast(bf16x8, u32x4{xh0, xh1, xl0, xl1});
}
struct YSplit {
  bf16x8 hh, l0;
};
__device__ __forceinline__ YSplit split_y(const f32x4& y) {
  const uint32_t yh0 = pack_bf2(y[0], y[1]), yh1 = pack_bf2(y[2], y[3]);
  const uint32_t yl0 = pack_bf2(y[0] - bf_lo(yh0), y[1] - bf_hi(yh0));
  const uint32_t yl1 = pack_bf2(y[2] - bf_lo(yh1), y[3] - bf_hi(yh1));
  return YSplit{__builtin_bit_cast(bf16x8, u32x4{yh0, yh1, yh0, yh1}),
                __builtin_bit_cast(bf16x8, u32x4{yl0, yl1, 0u, 0u})};
}
__device__ __forceinline__ f32x4 prod16(const bf16x8& xa, const YSplit& y, f32x4 acc) {
  acc = mfma16(xa, y.hh, acc);
  return mfma16(xa, y.l0, acc);
}

// Wave-local LDS hand-off between lanes of one wave: LDS operations of a wave
// complete in order; this keeps the compiler from moving them across.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One lane's 16 bytes of a fragment: streamed to global memory (read once, by
// the consumer), or a plain LDS store.
template <bool kToLds>
__device__ __forceinline__ void store_frag(const u32x4& x, uint16_t* dst) {
  if constexpr (kToLds) {
    *reinterpret_cast<u32x4*>(dst) = x;
  } else {
    __builtin_nontemporal_store(x, reinterpret_cast<u32x4*>(dst));
  }
}

// The terms of NH v-heads (one, or both of a GVA pair, interleaved phase by
// phase so that their independent latency chains overlap) from the chunk's raw
// gram: kk[m][n] (n <= m) holds [t = 16 m + 4 lg + rr][i = 16 n + l16] =
// k_t . k_i.  a_t, b_t: this lane's token (clamped into the chunk) per v-head.
// The terms (Tb fragments; gam, tail, the map bound and Gam in the gate block)
// go to frag0 / gp0 in the workspace layout: global memory (streamed out), or
// LDS when kToLds (the direct path).  Aqk is formed by the consumers, from the
// K / Q rows they hold anyway.  NB: the number of 16-token blocks that hold
// tokens (c <= 16 NB).  Later blocks have beta = 0, so their rows of N and
// every fragment of Tb that touches them are exactly zero: they are stored as
// zeros without being formed.  Two phases: prepass_gates, then prepass_terms.
//
// The gates of NH v-heads (the first phase of the terms; it needs only a, b
// and the per-head constants, so it can run while the chunk's K rows are in
// flight): Gam_t = inclusive scan of log2 g (clamped: g = e^-100 is already 0
// to fp32 working precision, and a finite floor keeps Gam finite), beta_t;
// gam / tail / Gam to the gate blocks, Gam and beta to ws rows 0 .. NH - 1,
// Gam at the chunk's last token to last[].
template <int NH, bool kToLds = false>
__device__ __forceinline__ void prepass_gates(PrepassWaveSmem& ws, int c, const float (&a_t)[kGva],
                                              const float (&b_t)[kGva], const float (&alog)[kGva],
                                              const float (&dtb)[kGva], float* __restrict__ gp0,
                                              float (&last)[NH]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int e = 0; e < NH; ++e) {
    // formed on every lane (a lane past the chunk holds its last token's
    // gates: finite), then masked: no branch for the compiler to sink the
    // gate loads into behind the K rows' loads
    const float lgv_all = fmaxf(log_decay(alog[e], a_t[e], dtb[e]), -100.0f) * kLog2e;
    const float bet_all = sigmoidf(b_t[e]);
    const float lgv = lane < c ? lgv_all : 0.0f;
    const float bet = lane < c ? bet_all : 0.0f;
    const float lgam = wave_incl_sumf(lgv);
    last[e] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lgam), c - 1));
    float* gp = gp0 + e * kGamStride;
    gp[lane] = lane < c ? fast_exp2(lgam) : 0.0f;
    gp[kChunk + lane] = lane < c ? fast_exp2(last[e] - lgam) : 0.0f;
    gp[kLgamAt + lane] = lgam;
    ws.lgam[e][lane] = lgam;
    ws.beta[e][lane] = bet;
  }
  wave_lds_sync();
}

// The rest of the terms of NH v-heads, whose gates prepass_gates left in ws
// rows E0 .. E0 + NH - 1 (and last[]), from the chunk's raw gram.
template <int NH, int E0 = 0, bool kToLds = false, int NB = 4>
__device__ __forceinline__ void prepass_terms(PrepassWaveSmem& ws, const f32x4 (&kk)[4][4], int c,
                                              const float (&last)[NH], uint16_t* __restrict__ frag0,
                                              float* __restrict__ gp0) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  // per-head workspace blocks are consecutive v-heads of one record
  constexpr size_t kFragStride = kMatElems;
  float lcol[NH][4];     // Gam at column 16 n + l16
  f32x4 lrow[NH][4];     // Gam at rows 16 m + 4 lg + rr
  f32x4 brow[NH][4];     // beta at rows 16 m + 4 lg + rr
#pragma unroll
  for (int e = 0; e < NH; ++e)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      lcol[e][m] = ws.lgam[E0 + e][16 * m + l16];
      lrow[e][m] = *reinterpret_cast<const f32x4*>(&ws.lgam[E0 + e][16 * m + 4 * lg]);
      brow[e][m] = *reinterpret_cast<const f32x4*>(&ws.beta[E0 + e][16 * m + 4 * lg]);
    }

  // ---- N = strict_lower(beta_t rho K K^T): diagonal tiles to LDS
  // (column-major) for the substitution, their diagonal |k_t|^2 into the
  // chunk's map bound; lower tiles stay in registers ----
  f32x4 nlo[NH][4][4];     // nlo[e][m][n], n < m
  float kb[NH];            // log2 max(1, |1 - beta_t |k_t|^2|) of the token this lane holds (else 0)
#pragma unroll
  for (int e = 0; e < NH; ++e) {
    kb[e] = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int n = 0; n <= m; ++n) {
        f32x4 nv;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int t = 16 * m + 4 * lg + rr, i = 16 * n + l16;
          nv[rr] = (m < NB && i < t) ? brow[e][m][rr] * fast_exp2(lrow[e][m][rr] - lcol[e][n]) * kk[m][n][rr] : 0.0f;
        }
        if (n == m) {
          // t = 16 m + l16 sits on the lane whose rows include it (rr = l16 - 4 lg);
          // rows t >= c have beta = 0 and contribute 0
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            if (m < NB && l16 == 4 * lg + rr) kb[e] += __log2f(fmaxf(1.0f, fabsf(1.0f - brow[e][m][rr] * kk[m][m][rr])));
          *reinterpret_cast<f32x4*>(&ws.nt[E0 + e][m][l16][4 * lg]) = nv;
        } else {
          nlo[e][m][n] = nv;
        }
      }
    }
  }
  wave_lds_sync();

  // ---- T_aa = (I + N_aa)^{-1} by forward substitution: lane (a = lg, j = l16)
  // forms column j of T_aa; once x[i] is final every later row subtracts
  // N[r][i] x[i] (the row-wise recurrence's terms and order, dependency depth 16) ----
  // the column index through an opaque move: otherwise the compiler hoists the
  // identity columns out of the item loop and spills them
  int jcol;
  asm volatile("v_and_b32 %0, 15, %1" : "=v"(jcol) : "v"(lane));
#pragma unroll
  for (int e = 0; e < NH; ++e) {
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = i == jcol ? 1.0f : 0.0f;
    // column i's quads are read three steps ahead into a ring (at most 12 LDS
    // reads in flight), so a step waits only for reads issued long before it
    // instead of one LDS round trip per step
    constexpr int kAhead = 3;
    f32x4 ring[kAhead][4];
    auto read_col = [&](int i, f32x4 (&c)[4]) {
#pragma unroll
      for (int qv = (i + 1) >> 2; qv < 4; ++qv) c[qv] = *reinterpret_cast<const f32x4*>(&ws.nt[E0 + e][lg][i][4 * qv]);
    };
#pragma unroll
    for (int i = 0; i < kAhead; ++i) read_col(i, ring[i]);
#pragma unroll
    for (int i = 0; i < 15; ++i) {
      f32x4 (&c)[4] = ring[i % kAhead];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rr = i + 1; rr < 16; ++rr) x[rr] = fmaf(-c[rr >> 2][rr & 3], x[i], x[rr]);
      __builtin_amdgcn_sched_barrier(0);
      if (i + kAhead < 15) read_col(i + kAhead, ring[i % kAhead]);
    }
#pragma unroll
    for (int qv = 0; qv < 4; ++qv)
      *reinterpret_cast<f32x4*>(&ws.nt[E0 + e][lg][l16][4 * qv]) = f32x4{x[4 * qv], x[4 * qv + 1], x[4 * qv + 2], x[4 * qv + 3]};
  }
  wave_lds_sync();

  // ---- W = T^T: diagonal blocks from LDS in both orientations, the
  // off-diagonal blocks by distance, then Tb^T = diag(beta) W (row i = 16 a +
  // 4 lg + rr) as fp16 fragments: fragment (m, d) slots 0-3 from tile (2 d, m),
  // slots 4-7 from (2 d + 1, m).  One v-head after the other (registers). ----
#pragma unroll
  for (int e = 0; e < NH; ++e) {
    f32x4 tc[4], w[4][4];   // tc[a] = T_aa = (W_aa)^T in C layout; w[a][b] = W_ab, a <= b
#pragma unroll
    for (int ab = 0; ab < 4; ++ab) {
      tc[ab] = *reinterpret_cast<const f32x4*>(&ws.nt[E0 + e][ab][l16][4 * lg]);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) w[ab][ab][rr] = ws.nt[E0 + e][ab][4 * lg + rr][l16];
    }
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    // operands split once: tx[a] from T_aa, nx[m][a] from N_ma = U_am^T,
    // wy[m][b] from W_mb (m >= 1: the rows above use it)
    bf16x8 tx[3], nx[4][3];
    YSplit wy[4][4];
#pragma unroll
    for (int a = 0; a < 3; ++a) tx[a] = split_x(tc[a]);
#pragma unroll
    for (int m = 1; m < 4; ++m) {
      wy[m][m] = split_y(w[m][m]);
#pragma unroll
      for (int a = 0; a < m; ++a) nx[m][a] = split_x(nlo[e][m][a]);
    }
#pragma unroll
    for (int dist = 1; dist < NB; ++dist) {
#pragma unroll
      for (int ab = 0; ab + dist < NB; ++ab) {
        const int bb = ab + dist;
        // P = sum_m U_am W_mb, the term of the block formed last (m = ab + 1)
        // added last, so only it waits for the previous distance
        f32x4 p = z4;
#pragma unroll
        for (int m = bb; m > ab; --m) p = prod16(nx[m][ab], wy[m][bb], p);
        w[ab][bb] = -prod16(tx[ab], split_y(p), z4);
        if (ab >= 1) wy[ab][bb] = split_y(w[ab][bb]);
      }
    }
    // Tb^T = diag(beta) W (row ai = 2 d + hf of fragment (m, d)).  Tb goes to
    // fp16 scaled by a power of two that puts the wave's largest |Tb| into
    // fp16's normal range when it is not there already (beta below about 6e-5
    // would otherwise leave fp16 subnormals); the consumers divide Delta = Tb R
    // by the same factor, whose inverse goes to the gate block.
    auto tb_val = [&](int m, int ai, int rr) {
      return (ai <= m && m < NB) ? brow[e][ai][rr] * w[ai][m][rr] : 0.0f;
    };
    float tmx = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int ai = 0; ai <= m; ++ai)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) tmx = fmaxf(tmx, fabsf(tb_val(m, ai, rr)));
    const float tsc = fp16_range_scale(tmx);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        if (frag_zero(m, d)) continue;
        float x[8];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) x[4 * hf + rr] = tb_val(m, 2 * d + hf, rr);
        if (tsc != 1.0f) {   // uniform
#pragma unroll
          for (int j = 0; j < 8; ++j) x[j] *= tsc;
        }
        store_frag<kToLds>(
            u32x4{pack_h2(x[0], x[1]), pack_h2(x[2], x[3]), pack_h2(x[4], x[5]), pack_h2(x[6], x[7])},
            frag0 + e * kFragStride + (frag_slot(m, d) * 64 + lane) * 8);
      }
    }
    if (lane == 0) gp0[e * kGamStride + kTbScaleAt] = 1.0f / tsc;   // exact: a power of two
  }

  // the chunk's map bound: sum over tokens of log2 g_t + log2 max(1, |1 - beta_t |k_t|^2|)
#pragma unroll
  for (int e = 0; e < NH; ++e) {
    const float lb = wave_sumf(kb[e]) + last[e];
    if (lane == 0) gp0[e * kGamStride + kBoundAt] = lb;
  }
}

// Raw gram of one chunk (rows t0 .. t0 + c - 1 of q/k head hq), one wave:
// kk = K K^T (lower tiles, kk[m][n] = [t = 16 m + 4 lg + rr][i = 16 n + l16]).
// Fragment (m, d) of a 64x128 row block: lane (lg, l16) holds row 16 m + l16,
// columns 32 d + 8 lg .. + 7.  Rows past the chunk end repeat row c - 1: they
// meet beta = 0 (rows of N) and i <= t masks.  Only the tiles of the first NB
// 16-row blocks are formed.
// The gram comes in two steps: every fragment of the chunk's K rows requested
// at once (one memory round trip; the gates are formed while they are in
// flight), then the products.
// ND: the depth chunks loaded into kf[0 .. ND - 1], from depth chunk d0 on
// (all four by default).  The gram sums over depth chunks, so the slot a
// depth chunk occupies does not matter as long as every slot holds one.
template <int NB = 4, int ND = 4>
__device__ __forceinline__ void chunk_gram_loads(const uint16_t* __restrict__ k, long long t0, int c, int hq,
                                                 int lane, bf16x8 (&kf)[4][4], int d0 = 0) {
  const int l16 = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int m = 0; m < NB; ++m) {
    const size_t row = static_cast<size_t>(t0 + min(16 * m + l16, c - 1));
    const uint16_t* krow = k + (row * kQKHeads + hq) * kDim + 8 * lg + 32 * d0;
#pragma unroll
    for (int dd = 0; dd < ND; ++dd) kf[dd][m] = *reinterpret_cast<const bf16x8*>(krow + 32 * dd);
  }
}

// The two waves of a GVA pair (items 2j, 2j + 1 of one record on adjacent
// waves of a work-group) each load half of the chunk's K fragments (depth
// chunks 2 (item & 1) and 2 (item & 1) + 1, into slots 0 and 1) and trade them
// through LDS into slots 2 and 3.  The exchange area is the wave's N-block
// area (8 KB, unused until the terms), fragment f = 4 slot + m at
// 16 (64 f + lane).  Two work-group barriers: the halves written, then read
// (before any terms overwrite them).  Every wave of the group takes part: in
// each pass of the item loop the group's four waves hold items 4i .. 4i + 3
// and the item count is a multiple of 8 (8 per record), so either all four
// have an item or none has, and a wave that has ended no longer counts at a
// barrier.
static_assert(sizeof(PrepassWaveSmem::nt) >= 8 * 64 * sizeof(u32x4), "the exchange area holds eight fragments");
__device__ __forceinline__ void trade_gram_halves(u32x4* mine, const u32x4* partner, int lane,
                                                  bf16x8 (&kf)[4][4]) {
#pragma unroll
  for (int f = 0; f < 8; ++f) mine[64 * f + lane] = __builtin_bit_cast(u32x4, kf[f >> 2][f & 3]);
  __syncthreads();
#pragma unroll
  for (int f = 0; f < 8; ++f) kf[2 + (f >> 2)][f & 3] = __builtin_bit_cast(bf16x8, partner[64 * f + lane]);
  __syncthreads();
}
template <int NB = 4>
__device__ __forceinline__ void chunk_gram_products(const bf16x8 (&kf)[4][4], f32x4 (&kk)[4][4]) {
  // the products wait for K: nothing formed before this point (the gates)
  // may be scheduled behind them
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < NB; ++m)
#pragma unroll
    for (int n = 0; n <= m; ++n) kk[m][n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int dd = 0; dd < 4; ++dd)
#pragma unroll
    for (int m = 0; m < NB; ++m)
#pragma unroll
      for (int n = 0; n <= m; ++n) kk[m][n] = mfma16(kf[dd][m], kf[dd][n], kk[m][n]);
}

// kGroups: work-groups per CU the register budget is sized for (2, or 3 for
// one-v-head items in batches of 2048-3072 of them).
template <bool kPair, int kGroups>
__global__ __launch_bounds__(kPrepassThreads, kGroups) void prepass_kernel(
    const uint16_t* __restrict__ k, const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b,
    const int4* __restrict__ recs, const void* __restrict__ cu, int is64, int num_seqs, long long T, int R,
    int gcap, int fused_plan, int* __restrict__ rec_start, int* __restrict__ lists,
    uint16_t* __restrict__ ws_frag, float* __restrict__ ws_gam) {
  __shared__ PrepassSmem sm;
  if (fused_plan && blockIdx.x == 0) {
    // work-group 0 plans the batch (lists for the consumer) while the others
    // run the records
    int total_recs;
    plan_batch<kPrepassThreads>(cu, is64, num_seqs, T, R, gcap, A_log, dt_bias, rec_start, lists, sm.u.plan,
                                total_recs);
    return;
  }
  const int lane = threadIdx.x & 63;
  // the per-head constants, requested first: lane l holds v-head l & 7's
  const float alog_l = A_log[lane & 7], dtb_l = dt_bias[lane & 7];
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  PrepassWaveSmem& ws = sm.u.w[wv];
  const int gw = (static_cast<int>(blockIdx.x) - fused_plan) * kPrepassWaves + wv;
  const int nw = (static_cast<int>(gridDim.x) - fused_plan) * kPrepassWaves;

  // records: small batches scan the chunk counts here (wave 0; lane l of block
  // j owns sequence 64 j + l), into LDS
  int total;
  if (fused_plan) {
    const int nblk = (num_seqs + 63) / 64;
    if (wv == 0) {
      // every block's bounds are requested before the first is scanned (one
      // memory round trip instead of one per block)
      // (lanes past the last sequence read a valid entry, then count as empty)
      long long b0[kFusedBlocks], b1[kFusedBlocks];
      if (is64) {
        const long long* c64 = static_cast<const long long*>(cu);
#pragma unroll
        for (int j = 0; j < kFusedBlocks; ++j) {
          const int i = min(64 * j + lane, num_seqs - 1);
          b0[j] = c64[i];
          b1[j] = c64[i + 1];
        }
      } else {
        const int* c32 = static_cast<const int*>(cu);
#pragma unroll
        for (int j = 0; j < kFusedBlocks; ++j) {
          const int i = min(64 * j + lane, num_seqs - 1);
          b0[j] = c32[i];
          b1[j] = c32[i + 1];
        }
      }
      int carry = 0;
#pragma unroll
      for (int j = 0; j < kFusedBlocks; ++j) {
        if (j < nblk) {
          const int s = 64 * j + lane;
          // the clamps of seq_bounds
          long long t0 = b0[j] < 0 ? 0 : (b0[j] > T ? T : b0[j]);
          long long t1 = b1[j] < t0 ? t0 : (b1[j] > T ? T : b1[j]);
          if (s >= num_seqs) t0 = t1 = 0;
          b0[j] = t0;
          b1[j] = t1;
          const int nch = static_cast<int>((b1[j] - b0[j] + kChunk - 1) / kChunk);
          const int inc = wave_incl_sum(nch) + carry;
          sm.seq.incl[s] = inc;
          sm.seq.s0[s] = b0[j];
          sm.seq.s1[s] = b1[j];
          carry = __builtin_amdgcn_readlane(inc, 63);
        }
      }
    }
    __syncthreads();
    total = min(sm.seq.incl[64 * nblk - 1], R);
  } else {
    total = min(rec_start[num_seqs], R);
  }

  // items: (record r, v-head h) = 8 r + h, or (record r, q/k head hq) = 4 r + hq
  // with both v-heads of the pair; consecutive items share a work-group, so the
  // waves that read the same K / Q rows go through one L2
  constexpr bool pair_items = kPair;
  const int per_rec = pair_items ? kQKHeads : kVHeads;
  const int nitems = total * per_rec;
  for (int item = gw; item < nitems; item += nw) {
    const int r = item / per_rec;
    const int hq = pair_items ? item % kQKHeads : (item % kVHeads) / kGva;
    const int e0 = pair_items ? 0 : item % kGva;       // first v-head of the pair this item runs
    const int ne = pair_items ? kGva : 1;
    long long t0, s1;
    if (fused_plan) {
      // the first sequence whose inclusive chunk count exceeds r (one exists: r < total)
      int s = 0, start = 0;
      for (int j = 0;; ++j) {
        const int inc = sm.seq.incl[64 * j + lane];
        const unsigned long long m = __builtin_amdgcn_ballot_w64(inc > r);
        if (m != 0) {
          const int l = static_cast<int>(__builtin_ctzll(m));
          s = 64 * j + l;
          start = s > 0 ? __builtin_amdgcn_readfirstlane(sm.seq.incl[s - 1]) : 0;
          break;
        }
      }
      const long long s0 = sm.seq.s0[s];
      s1 = sm.seq.s1[s];
      t0 = s0 + static_cast<long long>(r - start) * kChunk;
    } else {
      const int4 rec = recs[r];
      t0 = rec.y;
      s1 = t0 + max(rec.z, 1);
    }
    const int c = static_cast<int>(min(static_cast<long long>(kChunk), s1 - t0));
    const int cm1 = c - 1;

    // ---- loads: gates (lane = token, clamped into the chunk), then every
    // fragment of the K rows (shared by the v-heads of the pair); the gates
    // are formed while K is in flight ----
    const size_t gi = static_cast<size_t>(t0 + min(lane, cm1)) * kVHeads + kGva * hq + e0;
    float a_t[kGva], b_t[kGva];
#pragma unroll
    for (int e = 0; e < kGva; ++e) {
      a_t[e] = e < ne ? bf2f(a[gi + e]) : 0.0f;
      b_t[e] = e < ne ? bf2f(b[gi + e]) : 0.0f;
    }
    bf16x8 kf[4][4];
    if constexpr (pair_items)
      chunk_gram_loads(k, t0, c, hq, lane, kf);
    else
      chunk_gram_loads<4, 2>(k, t0, c, hq, lane, kf, 2 * e0);

    const int h0 = kGva * hq + e0;
    float alog[kGva], dtb[kGva];
#pragma unroll
    for (int e = 0; e < kGva; ++e) {
      const int hh = min(h0 + e, kVHeads - 1);
      alog[e] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alog_l), hh));
      dtb[e] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dtb_l), hh));
    }
    uint16_t* frag0 = ws_frag + (static_cast<size_t>(r) * kVHeads + h0) * kMatElems;
    float* gp0 = ws_gam + (static_cast<size_t>(r) * kVHeads + h0) * kGamStride;
    f32x4 kk[4][4];
    if constexpr (pair_items) {
      float last[kGva];
      prepass_gates<kGva>(ws, c, a_t, b_t, alog, dtb, gp0, last);
      chunk_gram_products(kf, kk);
      // the v-heads of the pair one after the other (interleaving their
      // phases gains nothing: the phases are VALU-bound, not latency-bound)
      const float l0[1] = {last[0]}, l1[1] = {last[1]};
      prepass_terms<1, 0>(ws, kk, c, l0, frag0, gp0);
      prepass_terms<1, 1>(ws, kk, c, l1, frag0 + kMatElems, gp0 + kGamStride);
    } else {
      float last[1];
      prepass_gates<1>(ws, c, a_t, b_t, alog, dtb, gp0, last);
      auto* mine = reinterpret_cast<u32x4*>(&ws.nt[0][0][0][0]);
      const auto* partner = reinterpret_cast<const u32x4*>(&sm.u.w[wv ^ 1].nt[0][0][0][0]);
      trade_gram_halves(mine, partner, lane, kf);
      chunk_gram_products(kf, kk);
      prepass_terms<1, 0>(ws, kk, c, last, frag0, gp0);
    }
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
//             is stored at position j ^ kq_swz(t) (row reads conflict-free,
//             transposed reads at two passes per 32 lanes).
//   vs      : V rows; chunk j of row t at j ^ v_swz(t).
//   frag    : Tb (fp16, copied) and Aqk (bf16, formed by the waves) in
//             permuted fragment order (lane-contiguous).
//   gt      : the gate block: gam[64], tail[64], the map bound, Gam[64].
// Rows t >= c of a partial chunk hold copies of row c-1 (finite data) or
// zeros; they only meet zero rows / columns of Tb and Aqk and zero gam / tail.
struct __align__(16) ConsumerSmem {
  uint16_t ks[2][kChunk][kDim];
  uint16_t qs[2][kChunk][kDim];
  uint16_t vs[2][kChunk][kDim];
  uint16_t frag[2][kFrags][kMatElems];
  float gt[2][4 * kChunk];
};

__device__ __forceinline__ int v_swz(int t) { return (t & 3) << 2; }

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

__device__ __forceinline__ f16x8 half_frag(const float (&x)[8]) {
  return __builtin_bit_cast(f16x8, u32x4{pack_h2(x[0], x[1]), pack_h2(x[2], x[3]),
                                         pack_h2(x[4], x[5]), pack_h2(x[6], x[7])});
}

__device__ __forceinline__ float r_scale(const f32x4 (&Rt)[4]) {
  float mx = 0.0f;
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) mx = fmaxf(mx, fabsf(Rt[m][rr]));
  return fp16_range_scale(mx);
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

// Aqk tile (a, m), a <= m: from the raw tile acc = K_a Q_m^T (C layout: lane
// (lg, l16) holds rows i = 16 a + 4 lg + rr of column t = 16 m + l16) forms
// lower(rho . acc), rho[t, i] = 2^(Gam_t - Gam_i), and writes it as slots
// 4 (a & 1) .. + 3 of Aqk fragment (m, a >> 1) in frag (an LDS Aqk matrix in
// permuted fragment order).  For even a on the diagonal it also zeroes slots
// 4-7, which would come from tile (a + 1, m) above the diagonal.  Rows of a
// partial chunk past its end only reach entries no stored output reads.
__device__ __forceinline__ void put_aqk_tile(uint16_t* frag, int a, int m, int lane, const f32x4& acc, float gam_t,
                                             const f32x4& gam_i) {
  const int l16 = lane & 15, lg = lane >> 4;
  const int t = 16 * m + l16;
  float x[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) x[rr] = 16 * a + 4 * lg + rr <= t ? fast_exp2(gam_t - gam_i[rr]) * acc[rr] : 0.0f;
  uint16_t* dst = frag + (frag_slot(m, a >> 1) * 64 + lane) * 8 + 4 * (a & 1);
  const uint32_t h0 = pack_bf2(x[0], x[1]), h1 = pack_bf2(x[2], x[3]);
  if ((a & 1) == 0 && a == m)
    *reinterpret_cast<u32x4*>(dst) = u32x4{h0, h1, 0u, 0u};
  else
    *reinterpret_cast<u32x2*>(dst) = u32x2{h0, h1};
}

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
    dma16<2>(vb + row * (kVHeads * kDim * 2) + dl.v_col, &sm.vs[P][32 * j + 4 * w][0]);   // read once
  }
  const size_t rh = static_cast<size_t>(cr.rec) * kVHeads + h;
  const char* fb = reinterpret_cast<const char*>(ws_frag + rh * kMatElems);
  // the 6 Tb fragments of 1 KB: wave w copies fragment w; waves 6-7 copy
  // fragments 0-1 again (the same bytes to the same place: branch-free).  The
  // waves form Aqk themselves (consumer_chunk).
  static_assert(kMatFrags == 6 && kConsumerWaves == 8, "fragment copy split");
  const int wf = w < kMatFrags ? w : w - kMatFrags;
  dma16<2>(fb + (64 * wf + lane) * 16, &sm.frag[P][0][0] + 64 * wf * 8);   // read once
  if (w == 0)   // the gate block (gam, tail, the map bound, Gam): 1 KB
    dma16(reinterpret_cast<const char*>(ws_gam + rh * kGamStride) + 16 * lane, &sm.gt[P][0]);
}

// Full-head consumer wave W's Aqk tiles (a, m) (put_aqk_tile): K row block a
// for waves 0-1 is 0, for 2-3 is 1, for 4-5 is 2, for 6 is 3; Q row blocks
// m0 (and m1).  Wave 7 forms none.  Every LDS read is issued before the first
// product.
__host__ __device__ constexpr int fh_aqk_a(int w) { return w < 2 ? 0 : w < 4 ? 1 : w < 6 ? 2 : w == 6 ? 3 : -1; }
__host__ __device__ constexpr int fh_aqk_m0(int w) {
  return w == 0 ? 0 : w == 1 ? 2 : w == 2 ? 1 : w == 3 ? 3 : w == 4 ? 2 : w < 7 ? 3 : -1;
}
__host__ __device__ constexpr int fh_aqk_m1(int w) { return w == 0 ? 1 : w == 1 ? 3 : w == 2 ? 2 : -1; }
constexpr bool fh_aqk_covers() {   // every tile a <= m exactly once, none above the diagonal
  int n[4][4] = {};
  for (int w = 0; w < kConsumerWaves; ++w) {
    if (fh_aqk_a(w) < 0) continue;
    ++n[fh_aqk_a(w)][fh_aqk_m0(w)];
    if (fh_aqk_m1(w) >= 0) ++n[fh_aqk_a(w)][fh_aqk_m1(w)];
  }
  for (int a = 0; a < 4; ++a)
    for (int m = 0; m < 4; ++m)
      if (n[a][m] != (a <= m ? 1 : 0)) return false;
  return true;
}
static_assert(fh_aqk_covers(), "full-head Aqk tiles");

// Tiles of Q row blocks at or past the chunk length c feed only output rows
// that are never stored: they are skipped (m1 > m0, so m0's test covers both).
template <int W, int P>
__device__ __forceinline__ void fh_aqk(ConsumerSmem& sm, int lane, int c) {
  constexpr int a = fh_aqk_a(W), m0 = fh_aqk_m0(W), m1 = fh_aqk_m1(W);
  static_assert(m1 < 0 || m1 > m0, "tile order");
  if constexpr (a >= 0) {
    if (16 * m0 >= c) return;   // uniform
    const int l16 = lane & 15, lg = lane >> 4;
    const int rsw = kq_swz(l16);
    bf16x8 kb[4], q0[4], q1[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int at = 8 * ((4 * d + lg) ^ rsw);
      kb[d] = *reinterpret_cast<const bf16x8*>(&sm.ks[P][16 * a + l16][at]);
      q0[d] = *reinterpret_cast<const bf16x8*>(&sm.qs[P][16 * m0 + l16][at]);
      if constexpr (m1 >= 0) q1[d] = *reinterpret_cast<const bf16x8*>(&sm.qs[P][16 * m1 + l16][at]);
    }
    const f32x4 gi = *reinterpret_cast<const f32x4*>(&sm.gt[P][kLgamAt + 16 * a + 4 * lg]);
    const float g0 = sm.gt[P][kLgamAt + 16 * m0 + l16];
    const float g1 = sm.gt[P][kLgamAt + 16 * (m1 >= 0 ? m1 : m0) + l16];
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      acc0 = mfma16(kb[d], q0[d], acc0);
      if constexpr (m1 >= 0) acc1 = mfma16(kb[d], q1[d], acc1);
    }
    put_aqk_tile(&sm.frag[P][1][0], a, m0, lane, acc0, g0, gi);
    if constexpr (m1 >= 0)
      if (16 * m1 < c) put_aqk_tile(&sm.frag[P][1][0], a, m1, lane, acc1, g1, gi);
  }
}

// Calls f with the number of 16-token tiles that hold a chunk's c >= 1 tokens,
// as a compile-time constant (uniform branch).
template <class F>
__device__ __forceinline__ void chunk_by_tiles(int c, F&& f) {
  switch ((c + 15) >> 4) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    default: f(std::integral_constant<int, 4>{}); break;
  }
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
//   NB  : 16-token tiles that hold tokens (c <= 16 NB).  Rows t >= c have
//         beta = 0 and gam = tail = 0, so the later tiles contribute nothing
//         (zero columns of Tb, zero rows of Delta); their products are not
//         formed (their R rows count as zero, also for R's range scale), and
//         the state update skips the second 32-token depth half when NB <= 2.
template <int P, int NB>
__device__ __forceinline__ void consumer_chunk(ConsumerSmem& sm, int c, f32x4 (&st)[8], int w,
                                               int lane, float scale, __amdgpu_buffer_rsrc_t orc,
                                               uint32_t ocol) {
  static_assert(NB >= 1 && NB <= 4, "token tiles");
  constexpr int ND = (NB + 1) / 2;   // 32-token depth halves that hold tokens
  const int l16 = lane & 15, lg = lane >> 4;
  // ---- this wave's Aqk tiles, first (fewest registers live); every wave
  // reads them after the barrier before O^T ----
  switch (w) {   // uniform
    case 0: fh_aqk<0, P>(sm, lane, c); break;
    case 1: fh_aqk<1, P>(sm, lane, c); break;
    case 2: fh_aqk<2, P>(sm, lane, c); break;
    case 3: fh_aqk<3, P>(sm, lane, c); break;
    case 4: fh_aqk<4, P>(sm, lane, c); break;
    case 5: fh_aqk<5, P>(sm, lane, c); break;
    case 6: fh_aqk<6, P>(sm, lane, c); break;
    default: break;
  }
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
    if (m >= NB) continue;
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
    Rt[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (m >= NB) continue;
    const u32x2 vw = lds_tr16(&sm.vs[P][16 * m + vrow][vat]);
    const float vv[4] = {bf_lo(vw.x), bf_hi(vw.x), bf_lo(vw.y), bf_hi(vw.y)};
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) Rt[m][rr] = vv[rr] - gam[m][rr] * X[m][rr];
  }
  const float rsc = r_scale(Rt);
  if (rsc != 1.0f) {
#pragma unroll
    for (int m = 0; m < 4; ++m) Rt[m] = Rt[m] * rsc;
  }
  f16x8 rf[2];
#pragma unroll
  for (int d = 0; d < ND; ++d) {
    float x[8];
    gather_slots(Rt, d, x);
    rf[d] = half_frag(x);
  }
  f32x4 D[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    D[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (m >= NB) continue;
#pragma unroll
    for (int d = 0; d < ND; ++d)
      if (!frag_zero(m, d))
        D[m] = mfma16h(*reinterpret_cast<const f16x8*>(&sm.frag[P][0][(frag_slot(m, d) * 64 + lane) * 8]), rf[d], D[m]);
  }
  const float tbi = sm.gt[P][kTbScaleAt];   // 1 / Tb's fp16 range scale (1 in the usual range)
  if (rsc != 1.0f || tbi != 1.0f) {
    const float inv = tbi / rsc;   // exact: powers of two
#pragma unroll
    for (int m = 0; m < 4; ++m) D[m] = D[m] * inv;
  }

  // ---- Delta as bf16 (output) and Delta' = tail Delta as hi + lo (state) ----
  bf16x8 dob[2], dh[2], dl[2];
  {
    f32x4 Dt[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
      Dt[m] = m < NB ? D[m] * *reinterpret_cast<const f32x4*>(&sm.gt[P][kChunk + 16 * m + 4 * lg]) : D[m];
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      float x[8];
      gather_slots(D, d, x);
      dob[d] = round_frag(x);
      gather_slots(Dt, d, x);
      split_frag(x, dh[d], dl[d]);
    }
  }

  // ---- O^T = scale (Y^T diag(gam) + Delta^T Aqk^T): lane (lg, l16) holds token
  //      16m + l16, value columns 4lg .. 4lg+3 -> one 8-byte store ----
  lds_barrier();   // every wave's Aqk tiles are in LDS
#pragma unroll
  for (int m = 0; m < NB; ++m) {
    f32x4 OT = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < ND; ++d)
      if (!frag_zero(m, d))
        OT = mfma16(dob[d], *reinterpret_cast<const bf16x8*>(&sm.frag[P][1][(frag_slot(m, d) * 64 + lane) * 8]), OT);
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
    for (int d = 0; d < ND; ++d) {
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

// Full-head consumer over the short-sequence list (sequences of at most one
// chunk): work item = (list entry, v-head), item i on work-group wg = i mod
// nwg (short_entry / short_head).  nwg and the work-group's linear id are
// multiples of 8 apart, so item i runs on XCD i % 8.  Items are software-pipelined so that the state and operand traffic
// of one item overlaps the compute of the previous one: item k computes from
// LDS buffer k & 1 and its state registers while item k+1's state loads and
// operand copies (into the other buffer) are in flight and item k+2's list
// entry is loaded.  Every wave's vector-memory operations retire in issue
// order, so at the start of item k's stage, "at most 9 outstanding" (the list
// entry of item k+1 and the 8 new_state stores of item k-1, all issued after
// item k's loads) means item k's state and copies have landed.
struct ShortItem {
  int s, h, rec, c;   // sequence, v-head, record (-1: no chunk), tokens
  long long c0;
};

// Item i of the short list -> (list entry, v-head).  Items run on work-group
// i mod nwg, whose XCD is i % 8.  Within each block of 16 items (two entries)
// XCD x takes both v-heads of q/k head x % 4 of one entry, so the two v-heads
// that read the same K / Q rows share an L2; a last odd entry keeps the plain
// order (entry i / 8, v-head i % 8).
__device__ __forceinline__ int short_entry(int i, int nseq) {
  const int blk = i >> 4;
  return 2 * blk + 1 < nseq ? 2 * blk + ((i & 7) >> 2) : i >> 3;
}
__device__ __forceinline__ int short_head(int i, int nseq) {
  return 2 * (i >> 4) + 1 < nseq ? 2 * (i & 3) + ((i >> 3) & 1) : i & 7;
}

// The list entry arrives in VGPRs (see entry() below) and becomes scalar here.
__device__ __forceinline__ ShortItem short_item(const int4& e, int item, int nseq) {
  ShortItem it;
  it.s = __builtin_amdgcn_readfirstlane(e.x);
  it.h = short_head(item, nseq);
  it.rec = __builtin_amdgcn_readfirstlane(e.y);
  const int zw = __builtin_amdgcn_readfirstlane(e.w);
  it.c = zw >> 16;
  it.c0 = static_cast<long long>(static_cast<unsigned>(__builtin_amdgcn_readfirstlane(e.z))) |
          (static_cast<long long>(zw & 0xffff) << 32);
  return it;
}

__device__ __forceinline__ void full_head_items(
    ConsumerSmem& sm, int wg, int nwg, const int4* __restrict__ list, int nseq,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ state, float scale, const uint16_t* __restrict__ ws_frag,
    const float* __restrict__ ws_gam, uint16_t* __restrict__ out, float* __restrict__ new_state) {
  const int nitems = nseq * kVHeads;
  if (wg >= nitems) return;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int vcol = 16 * w;                       // first value row of this wave's tile
  DmaLane dl;
  {
    const int r = 4 * w + (lane >> 4);     // + 32 j keeps r & 15
    dl.row = r;
    dl.kq_col = 16u * static_cast<uint32_t>((lane & 15) ^ kq_swz(r));
    dl.v_col = 16u * static_cast<uint32_t>((lane & 15) ^ v_swz(r));
  }
  const uint32_t ocol = 2u * static_cast<uint32_t>(vcol + 4 * lg);
  auto kappa0 = [](int kt) { return 32 * (kt >> 1) + 4 * (kt & 1); };
  // state tile in the kappa k order (see consumer_chunk)
  auto st_off = [&](const ShortItem& it) {
    return ((static_cast<size_t>(it.s) * kVHeads + it.h) * kDim + vcol + l16) * kDim + 8 * lg;
  };
  auto load_state = [&](const ShortItem& it, f32x4 (&st)[8]) {
    if (state != nullptr && it.c > 0) {
      const float* sp = state + st_off(it);
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) st[kt] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sp + kappa0(kt)));
    } else {
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto issue = [&](const ShortItem& it, f32x4 (&st)[8], auto PC) {
    constexpr int P = decltype(PC)::value;
    load_state(it, st);
    if (it.rec >= 0 && it.c > 0)
      dma_chunk<P>(sm, ChunkRef{it.c0, it.c, it.rec}, dl, w, lane, it.h, it.h / kGva, q, k, v, ws_frag, ws_gam);
  };
  // the list entry of item i (a valid entry past the end keeps one load per
  // stage).  An opaque zero makes the address lane-varying, so the entry stays
  // in VGPRs until short_item() reads it one stage later: waiting for it then
  // does not wait for the loads and copies issued after it.
  int zero_v;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero_v));
  auto entry = [&](int i) { return list[short_entry(i < nitems ? i : 0, nseq) + zero_v]; };

  int item = wg;
  ShortItem cur = short_item(entry(item), item, nseq);
  f32x4 st[8];
  issue(cur, st, std::integral_constant<int, 0>{});
  int4 enext = entry(item + nwg);
  __builtin_amdgcn_s_waitcnt(0);

  // one item from buffer P; returns false after the group's last item
  auto stage = [&](auto PC) -> bool {
    constexpr int P = decltype(PC)::value;
    __builtin_amdgcn_s_waitcnt(0x0f79);   // vmcnt(9): this item's state and copies have landed
    lds_barrier();                         // ... in every wave
    const int inext = item + nwg;
    const bool has_next = inext < nitems;
    const ShortItem nx = short_item(enext, inext, nseq);
    f32x4 stn[8];
    if (has_next) issue(nx, stn, std::integral_constant<int, P ^ 1>{});
    enext = entry(inext + nwg);
    if (cur.rec >= 0 && cur.c > 0) {
      const __amdgpu_buffer_rsrc_t orc = __builtin_amdgcn_make_buffer_rsrc(
          out + (static_cast<size_t>(cur.c0) * kVHeads + cur.h) * kDim, 0, cur.c * (kVHeads * kDim * 2), 0x00020000);
      // all four tiles: batches of many short sequences are bound by their
      // state traffic, and one body keeps the loop's code small
      consumer_chunk<P, 4>(sm, cur.c, st, w, lane, scale, orc, ocol);
    }
    // an empty sequence leaves new_state zero (st is zero); a chunk without a
    // record (malformed cu_seqlens) passes the state through.  State bytes are
    // read and written once: non-temporal, as in decode.
    float* dst = new_state + st_off(cur);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) __builtin_nontemporal_store(st[kt], reinterpret_cast<f32x4*>(dst + kappa0(kt)));
    lds_barrier();   // buffer P is free for item k+2's copies
    if (!has_next) return false;
    item = inext;
    cur = nx;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) st[kt] = stn[kt];
    return true;
  };
  while (stage(std::integral_constant<int, 0>{}) && stage(std::integral_constant<int, 1>{})) {
  }
}

// ============================================================================
// direct path: calls of at most two chunks in total (T <= 128)
// ============================================================================
// Every sequence then has at most two chunks and the call is latency-bound, so
// it runs as one launch with no plan and no workspace: one work-group per
// (sequence, v-head).  All waves issue their share of the chunks' K / Q / V
// copies (chunk j into buffer j) and load their state tile; wave j then forms
// chunk j's terms (the prepass of one item, written to LDS instead of the
// workspace) while those land, and the eight waves run the chunks one after
// the other as the full-head consumer does, the state staying in registers.
constexpr int kDirectMaxSeqs = 64;
constexpr int kDirectMaxChunks = 2;

struct DirectSmem {
  ConsumerSmem c;                         // chunk j's operands in buffer j
  PrepassWaveSmem w[kDirectMaxChunks];    // scratch of the terms waves
};

__global__ __launch_bounds__(kConsumerThreads) void direct_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ state, const float* __restrict__ A_log, const uint16_t* __restrict__ a,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ b, const void* __restrict__ cu, int is64,
    long long T, float scale, uint16_t* __restrict__ out, float* __restrict__ new_state) {
  __shared__ DirectSmem sm;
  const int s = static_cast<int>(blockIdx.x) / kVHeads;
  const int h = static_cast<int>(blockIdx.x) % kVHeads;
  const int hq = h / kGva;
  long long t0, t1;
  seq_bounds(cu, is64, s, T, t0, t1);
  const int len = static_cast<int>(t1 - t0);   // 0 .. T <= 128
  const int nch = (len + kChunk - 1) / kChunk;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int vcol = 16 * w;
  auto kappa0 = [](int kt) { return 32 * (kt >> 1) + 4 * (kt & 1); };
  const size_t soff = ((static_cast<size_t>(s) * kVHeads + h) * kDim + vcol + l16) * kDim + 8 * lg;
  float* dst = new_state + soff;
  if (len <= 0) {   // an empty sequence: zero state, no output rows
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<f32x4*>(dst + kappa0(kt)));
    return;
  }
  // chunk j: first token t0 + 64 j, c_j tokens
  auto chunk_len = [&](int j) { return min(kChunk, len - kChunk * j); };
  // chunk j's K / Q / V rows into buffer j (rows past c_j repeat its last row)
  auto copy = [&](auto JC) {
    constexpr int J = decltype(JC)::value;
    const int r = 4 * w + (lane >> 4);
    const uint32_t kq_col = 16u * static_cast<uint32_t>((lane & 15) ^ kq_swz(r));
    const uint32_t v_col = 16u * static_cast<uint32_t>((lane & 15) ^ v_swz(r));
    const long long c0 = t0 + static_cast<long long>(kChunk) * J;
    const size_t qk0 = (static_cast<size_t>(c0) * kQKHeads + hq) * kDim;
    const char* kb = reinterpret_cast<const char*>(k + qk0);
    const char* qb = reinterpret_cast<const char*>(q + qk0);
    const char* vb = reinterpret_cast<const char*>(v + (static_cast<size_t>(c0) * kVHeads + h) * kDim);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const uint32_t row = static_cast<uint32_t>(min(r + 32 * jj, chunk_len(J) - 1));
      const uint32_t off = row * (kQKHeads * kDim * 2) + kq_col;
      dma16(kb + off, &sm.c.ks[J][32 * jj + 4 * w][0]);
      dma16(qb + off, &sm.c.qs[J][32 * jj + 4 * w][0]);
      dma16<2>(vb + row * (kVHeads * kDim * 2) + v_col, &sm.c.vs[J][32 * jj + 4 * w][0]);
    }
  };
  copy(std::integral_constant<int, 0>{});
  if (nch > 1) copy(std::integral_constant<int, 1>{});
  f32x4 st[8];
  if (state != nullptr) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
      st[kt] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(state + soff + kappa0(kt)));
  } else {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // wave j < nch forms chunk j's terms into buffer j
  auto terms = [&](auto JC) {
    constexpr int J = decltype(JC)::value;
    const int c = chunk_len(J);
    const long long c0 = t0 + static_cast<long long>(kChunk) * J;
    const size_t gi = static_cast<size_t>(c0 + min(lane, c - 1)) * kVHeads + h;
    const float a1[kGva] = {bf2f(a[gi]), 0.0f}, b1[kGva] = {bf2f(b[gi]), 0.0f};
    const float al1[kGva] = {A_log[h], 0.0f}, dt1[kGva] = {dt_bias[h], 0.0f};
    // only the 16-token blocks that hold tokens are formed (c <= 16 nb)
    auto blocks = [&](auto NBC) {
      constexpr int NB = decltype(NBC)::value;
      bf16x8 kf[4][4];
      chunk_gram_loads<NB>(k, c0, c, hq, lane, kf);
      float last[1];
      prepass_gates<1, true>(sm.w[J], c, a1, b1, al1, dt1, &sm.c.gt[J][0], last);
      f32x4 kk[4][4];
      chunk_gram_products<NB>(kf, kk);
      prepass_terms<1, 0, true, NB>(sm.w[J], kk, c, last, &sm.c.frag[J][0][0], &sm.c.gt[J][0]);
    };
    switch ((c + 15) >> 4) {
      case 1: blocks(std::integral_constant<int, 1>{}); break;
      case 2: blocks(std::integral_constant<int, 2>{}); break;
      case 3: blocks(std::integral_constant<int, 3>{}); break;
      default: blocks(std::integral_constant<int, 4>{}); break;
    }
  };
  if (w == 0) terms(std::integral_constant<int, 0>{});
  if (w == 1 && nch > 1) terms(std::integral_constant<int, 1>{});
  __builtin_amdgcn_s_waitcnt(0);   // copies, state loads and the terms have landed
  __syncthreads();
  const uint32_t ocol = 2u * static_cast<uint32_t>(vcol + 4 * lg);
  auto out_rsrc = [&](int j) {
    return __builtin_amdgcn_make_buffer_rsrc(out + ((static_cast<size_t>(t0) + kChunk * j) * kVHeads + h) * kDim, 0,
                                             chunk_len(j) * (kVHeads * kDim * 2), 0x00020000);
  };
  // each wave carries its own state tile: no barrier between the chunks
  if (nch > 1) {
    consumer_chunk<0, 4>(sm.c, chunk_len(0), st, w, lane, scale, out_rsrc(0), ocol);
    consumer_chunk<1, 4>(sm.c, chunk_len(1), st, w, lane, scale, out_rsrc(1), ocol);
  } else {
    // a lone chunk (short prompts): only its tiles that hold tokens
    chunk_by_tiles(chunk_len(0), [&](auto NBC) {
      consumer_chunk<0, decltype(NBC)::value>(sm.c, chunk_len(0), st, w, lane, scale, out_rsrc(0), ocol);
    });
  }
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) __builtin_nontemporal_store(st[kt], reinterpret_cast<f32x4*>(dst + kappa0(kt)));
}

// ============================================================================
// split consumer: one work-group per (seq, v-head, half of the value rows)
// ============================================================================
// For sequences of several chunks the recurrence is a chain through the state,
// so the time per chunk bounds the whole call.  Each 16-wide value tile gets
// two waves on one SIMD: the chain wave (waves 0-3) carries the state through
// X = K S^T, R, Delta = Tb R and S' = gam_c S + K^T Delta'; the side wave
// (waves 4-7) forms the chunk's Aqk tiles and the outputs (Y^T = S Q^T,
// O^T = Delta^T Aqk^T, stores) and copies the next chunk's operands.  The
// chain wave hands S and Delta (bf16 fragments, in its own register order) to
// its side wave through LDS, so the side wave's MFMAs and VALU work run in the
// gaps of the chain's dependent MFMA sequence.  Two barriers per chunk: B2
// (Delta and the Aqk tiles ready; waits for LDS traffic only, so the operand
// copies, issued at the chunk's start, stay in flight) and B3 at the chunk's
// end (see split_barrier).  The S fragments of chunk i+1 are written after
// B2 of chunk i, and the side wave reads them before B2 of chunk i+1, so one
// buffer suffices.
constexpr int kSplitThreads = 512;
constexpr int kHalfV = 64;                 // value rows per split work-group (4 tiles)
constexpr int kSideStores = 4;             // output stores a side wave issues per chunk, after its copies
static_assert(kSideStores == kChunk / 16, "side_chunk stores one 8-byte row piece per 16-token block");

// Barrier of the split consumer: every wave's LDS writes are visible, and each
// side wave has at most kPending vector memory operations outstanding.  The
// chain waves issue no vector memory operation a later phase depends on: their
// state loads are waited for where the state is first used, and their
// final-state stores need not have completed for the next item to start.
// At the chunk's end (B3), kPending = kSideStores: a side wave issues its
// copies at the chunk's start and its kSideStores output stores at the end,
// and vector memory operations complete in issue order, so every copy has
// landed while the output stores stay in flight into the next chunk.
template <int kPending>
__device__ __forceinline__ void split_barrier(bool chain) {
  static_assert(kPending >= 0 && kPending < 16, "vmcnt field");
  asm volatile("" ::: "memory");
  if (chain)
    __builtin_amdgcn_s_waitcnt(0xc07f);             // lgkmcnt(0)
  else
    __builtin_amdgcn_s_waitcnt(0x0070 | kPending);  // vmcnt(kPending), lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

struct __align__(16) SplitSmem {
  uint16_t ks[2][kChunk][kDim];
  uint16_t qs[2][kChunk][kDim];
  uint16_t vs[2][kChunk][kHalfV];          // this half's value columns; chunk j of row t at j ^ vh_swz(t)
  uint16_t frag[2][kFrags][kMatElems];
  float gt[2][4 * kChunk];
  u32x4 sbx[4][4][64];                     // chain wave w: bf16 S fragments sb[d], per lane
  u32x4 dox[4][2][64];                     // chain wave w: bf16 Delta fragments dob[d], per lane
  int next_item;                           // the group's next work item (from the queue)
};

__device__ __forceinline__ int vh_swz(int t) { return ((t >> 1) & 1) << 2; }

// Buffer resource over [base, base + bytes): loads past the end return zeros
// and stores past it are dropped by the hardware range check.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// 16 bytes per lane through a buffer resource straight into LDS (lane i of the
// wave writes bytes [16 i, 16 i + 16) after the wave-uniform LDS address).
// AUX is the cache policy of the load: 2 (nt) streams data read exactly once.
template <int AUX = 0>
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voff, void* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds_wave_base, 16,
                                           voff, 0, 0, AUX);
}

// Per-lane byte offsets of the side-wave copies; chunk-invariant because each
// chunk's base address lives in the (scalar) buffer resource.
struct SplitDmaLane {
  uint32_t kq[4];     // K / Q row (kr + 16 j), source chunk of this lane
  uint32_t v[2];      // V row (vr + 32 j), this half's source chunk
  uint32_t fr;        // fragment bytes of pass 0 (+4 KB per pass)
  uint32_t g;         // gate block
};

__device__ __forceinline__ SplitDmaLane split_dma_lane(int ws, int lane, int hv) {
  SplitDmaLane o;
  const int kr = 4 * ws + (lane >> 4);    // + 16 j keeps kr & 15
  const uint32_t kcol = 16u * static_cast<uint32_t>((lane & 15) ^ kq_swz(kr));
#pragma unroll
  for (int j = 0; j < 4; ++j) o.kq[j] = static_cast<uint32_t>(kr + 16 * j) * (kQKHeads * kDim * 2) + kcol;
  const int vr = 8 * ws + (lane >> 3);    // + 32 j keeps vr & 3
  const uint32_t vcol = 2u * kHalfV * hv + 16u * static_cast<uint32_t>((lane & 7) ^ vh_swz(vr));
#pragma unroll
  for (int j = 0; j < 2; ++j) o.v[j] = static_cast<uint32_t>(vr + 32 * j) * (kVHeads * kDim * 2) + vcol;
  o.fr = static_cast<uint32_t>(64 * ws + lane) * 16u;
  o.g = 16u * static_cast<uint32_t>(lane);
  return o;
}

// Side-wave copies of one chunk's operands into buffer P (4 side waves).
// Rows t >= c fall outside the K / Q / V resources and arrive as zeros.
template <int P>
__device__ __forceinline__ void split_dma(SplitSmem& sm, const ChunkRef& cr, const SplitDmaLane& dl, int ws,
                                          int h, int hq, bool zero_v, const uint16_t* __restrict__ q,
                                          const uint16_t* __restrict__ k,
                                          const uint16_t* __restrict__ v,
                                          const uint16_t* __restrict__ ws_frag,
                                          const float* __restrict__ ws_gam) {
  const size_t qk0 = (static_cast<size_t>(cr.c0) * kQKHeads + hq) * kDim;
  const uint32_t kq_bytes = static_cast<uint32_t>(cr.c) * (kQKHeads * kDim * 2);
  const __amdgpu_buffer_rsrc_t kr = buf_rsrc(k + qk0, kq_bytes);
  const __amdgpu_buffer_rsrc_t qr = buf_rsrc(q + qk0, kq_bytes);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    dma16_buf(kr, dl.kq[j], &sm.ks[P][16 * j + 4 * ws][0]);
    dma16_buf(qr, dl.kq[j], &sm.qs[P][16 * j + 4 * ws][0]);
  }
  // an M-run reads V = 0: an empty resource makes every V copy a zero fill
  const __amdgpu_buffer_rsrc_t vr = buf_rsrc(v + (static_cast<size_t>(cr.c0) * kVHeads + h) * kDim,
                                             zero_v ? 0u : static_cast<uint32_t>(cr.c) * (kVHeads * kDim * 2));
#pragma unroll
  for (int j = 0; j < 2; ++j) dma16_buf<2>(vr, dl.v[j], &sm.vs[P][32 * j + 8 * ws][0]);   // V: read once
  const size_t rh = static_cast<size_t>(cr.rec) * kVHeads + h;
  // the 6 Tb fragments of 1 KB: side wave ws copies ws and ws + 4 (< 6); the
  // side waves form Aqk themselves
  const __amdgpu_buffer_rsrc_t fr = buf_rsrc(ws_frag + rh * kMatElems, kMatElems * 2);
  dma16_buf(fr, dl.fr, &sm.frag[P][0][0] + 64 * ws * 8);
  if (ws + 4 < kMatFrags) dma16_buf(fr, dl.fr + 4096u, &sm.frag[P][0][0] + (256 + 64 * ws) * 8);
  if (ws == 0) dma16_buf(buf_rsrc(ws_gam + rh * kGamStride, kGamStride * 4), dl.g, &sm.gt[P][0]);
}

// bf16 B-operand fragments of the state tile: slots of depth chunk d are
// st[2d + s/4][s%4] (k = 32 d + 8 lg + s in the kappa order).
__device__ __forceinline__ void state_frags(const f32x4 (&st)[8], bf16x8 (&sb)[4]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float x[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) x[s] = st[2 * d + (s >> 2)][s & 3];
    sb[d] = round_frag(x);
  }
}

// The bf16 rounding residues of those fragments (lo = bf16(x - hi)).
__device__ __forceinline__ void state_frags_lo(const f32x4 (&st)[8], const bf16x8 (&hi)[4], bf16x8 (&lo)[4]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const u32x4 h = __builtin_bit_cast(u32x4, hi[d]);
    u32x4 l;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = 2 * j;
      l[j] = pack_bf2(st[2 * d + (s >> 2)][s & 3] - bf_lo(h[j]), st[2 * d + ((s + 1) >> 2)][(s + 1) & 3] - bf_hi(h[j]));
    }
    lo[d] = __builtin_bit_cast(bf16x8, l);
  }
}

// Chain wave, one chunk: S^T tile st (kappa k order, as in consumer_chunk).
// Each phase issues all of its LDS operand reads before its first product and
// runs its products over independent accumulators, so neither the LDS latency
// nor the MFMA result latency is paid per product.
template <int P>
__device__ __forceinline__ void chain_chunk(SplitSmem& sm, int c, f32x4 (&st)[8], int w, int lane) {
  const int l16 = lane & 15, lg = lane >> 4;
  const int rsw = kq_swz(l16);
  const int vrow = 4 * lg + (l16 >> 2);
  const int vat = 8 * ((2 * w + ((l16 & 3) >> 1)) ^ vh_swz(vrow)) + 4 * (l16 & 1);

  // ---- X = K S^T.  S enters as one bf16, plus its bf16 rounding residue
  // in a second pass when the chunk's map bound says the state barely decays:
  // then the rounding of S here is what accumulates over a long sequence
  // (single bf16: state error 1.2e-3 to 1.5e-3 at 4k to 28k tokens of near-1
  // decay; hi + lo: 3e-4 to 4e-4).  Where the map contracts by 2^-8 or more
  // per chunk, earlier roundings do not accumulate and one bf16 suffices.
  // The K fragments are read in two batches of eight and the products of a
  // depth chunk start once its fragments have landed (at most 15 LDS reads
  // can be waited for individually); the bound, read first, is tested after
  // the first pass.
  const float cbound = sm.gt[P][kBoundAt];   // first LDS read: done before the first K fragment
  const float tbi = sm.gt[P][kTbScaleAt];    // 1 / Tb's fp16 range scale (1 in the usual range)
  bf16x8 ka[4][4];
  auto read_k = [&](int d) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
      ka[d][m] = *reinterpret_cast<const bf16x8*>(&sm.ks[P][16 * m + l16][8 * ((4 * d + lg) ^ rsw)]);
  };
  read_k(0);
  read_k(1);
  bf16x8 sb[4];
  state_frags(st, sb);
  __builtin_amdgcn_sched_barrier(0);
  f32x4 X[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) X[m] = mfma16(ka[0][m], sb[0], f32x4{0.f, 0.f, 0.f, 0.f});
  __builtin_amdgcn_sched_barrier(0);
  read_k(2);
  read_k(3);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < 4; ++m) X[m] = mfma16(ka[1][m], sb[1], X[m]);
#pragma unroll
  for (int m = 0; m < 4; ++m) X[m] = mfma16(ka[2][m], sb[2], X[m]);
  __builtin_amdgcn_sched_barrier(0);
  // operands of R = V - gam X and the chunk's map bound
  f32x4 gam[4];
  u32x2 vw[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    gam[m] = *reinterpret_cast<const f32x4*>(&sm.gt[P][16 * m + 4 * lg]);
    vw[m] = lds_tr16(&sm.vs[P][16 * m + vrow][vat]);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < 4; ++m) X[m] = mfma16(ka[3][m], sb[3], X[m]);
  if (cbound > kHiLoBoundLog2) {   // uniform
    bf16x8 sbl[4];
    state_frags_lo(st, sb, sbl);
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int m = 0; m < 4; ++m) X[m] = mfma16(ka[d][m], sbl[d], X[m]);
  }
  // Tb fragments land while X runs
  f16x8 tb[2][4];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int m = 0; m < 4; ++m)
      if (!frag_zero(m, d)) tb[d][m] = *reinterpret_cast<const f16x8*>(&sm.frag[P][0][(frag_slot(m, d) * 64 + lane) * 8]);
  __builtin_amdgcn_sched_barrier(0);

  // ---- R = V - gam X, Delta = Tb R (fp16) ----
  f32x4 Rt[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float vv[4] = {bf_lo(vw[m].x), bf_hi(vw[m].x), bf_lo(vw[m].y), bf_hi(vw[m].y)};
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) Rt[m][rr] = vv[rr] - gam[m][rr] * X[m][rr];
  }
  const float rsc = r_scale(Rt);
  if (rsc != 1.0f) {
#pragma unroll
    for (int m = 0; m < 4; ++m) Rt[m] = Rt[m] * rsc;
  }
  f16x8 rf[2];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    float x[8];
    gather_slots(Rt, d, x);
    rf[d] = half_frag(x);
  }
  f32x4 D[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) D[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int m = 0; m < 4; ++m)
      if (!frag_zero(m, d)) D[m] = mfma16h(tb[d][m], rf[d], D[m]);
  if (rsc != 1.0f || tbi != 1.0f) {
    const float inv = tbi / rsc;   // exact: powers of two
#pragma unroll
    for (int m = 0; m < 4; ++m) D[m] = D[m] * inv;
  }

  // operands of the state update, read while Delta forms: tail gates and the
  // K^T fragments (tile kt, row i of the A operand is k = kappa(kt, i/4, i%4);
  // lane sl of group lg addresses K[t][k0 .. k0+3], t = perm_depth(d, lg, sl/4)
  // (+16 for slots 4..7), k0 = 32 (kt >> 1) + 8 (sl & 3) + 4 (kt & 1))
  f32x4 tl[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) tl[m] = *reinterpret_cast<const f32x4*>(&sm.gt[P][kChunk + 16 * m + 4 * lg]);
  const float gam_c = sm.gt[P][c - 1];
  const int sl = l16;
  const int tsw = kq_swz(4 * lg + (sl >> 2));
  bf16x8 kta[2][8];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const int ta = perm_depth(d, lg, sl >> 2);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      const int at = 8 * ((4 * (kt >> 1) + (sl & 3)) ^ tsw) + 4 * (kt & 1);
      kta[d][kt] = join_frag(lds_tr16(&sm.ks[P][ta][at]), lds_tr16(&sm.ks[P][ta + 16][at]));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    float x[8];
    gather_slots(D, d, x);
    sm.dox[w][d][lane] = __builtin_bit_cast(u32x4, round_frag(x));
  }
  lds_barrier();   // B2: Delta fragments visible to the side wave (and S fragments consumed)

  // ---- Delta' = tail Delta (hi + lo); S^T <- gam_c S^T + K^T Delta' ----
  bf16x8 dh[2], dl[2];
  {
    f32x4 Dt[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) Dt[m] = D[m] * tl[m];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      float x[8];
      gather_slots(Dt, d, x);
      split_frag(x, dh[d], dl[d]);
    }
  }
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) st[kt] = st[kt] * gam_c;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) st[kt] = mfma16(kta[d][kt], dh[d], st[kt]);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) st[kt] = mfma16(kta[d][kt], dl[d], st[kt]);
  }
  // S fragments of the next chunk for the side wave (read before its next B2)
  bf16x8 nb[4];
  state_frags(st, nb);
#pragma unroll
  for (int d = 0; d < 4; ++d) sm.sbx[w][d][lane] = __builtin_bit_cast(u32x4, nb[d]);
}

// The side wave that forms Aqk tile (a, m) (K row block a, Q row block m,
// a <= m): the ten tiles in row order go 3 / 3 / 2 / 2 to side waves 0-3, so
// no wave needs more than two K row blocks.
__host__ __device__ constexpr int aqk_owner(int a, int m) {
  const int idx = 4 * a - a * (a - 1) / 2 + (m - a);
  return idx < 3 ? 0 : idx < 6 ? 1 : idx < 8 ? 2 : 3;
}
constexpr bool aqk_owner_blocks() {   // side wave w's tiles use K row blocks max(w - 1, 0) and w only
  for (int a = 0; a < 4; ++a)
    for (int m = a; m < 4; ++m) {
      const int w = aqk_owner(a, m);
      if (w < 0 || w > 3 || (a != w && a != (w > 0 ? w - 1 : 0))) return false;
    }
  return true;
}
static_assert(aqk_owner_blocks(), "Aqk tile owners");

// Side wave WS, first half of a chunk: Y^T = S Q^T for chain wave WS's tile,
// and the wave's Aqk tiles (put_aqk_tile).  One straight-line body per wave:
// every LDS read is issued before the first product, and the Y^T and Aqk
// products interleave.
template <int WS, int P>
__device__ __forceinline__ void side_front(SplitSmem& sm, int lane, f32x4 (&YT)[4]) {
  const int l16 = lane & 15, lg = lane >> 4;
  const int rsw = kq_swz(l16);
  constexpr int a_lo = WS > 0 ? WS - 1 : 0;   // the K row blocks this wave's tiles use
  constexpr int a_hi = WS;
  bf16x8 sb[4], qa[4][4], kb[2][4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    sb[d] = __builtin_bit_cast(bf16x8, sm.sbx[WS][d][lane]);
#pragma unroll
    for (int m = 0; m < 4; ++m)
      qa[d][m] = *reinterpret_cast<const bf16x8*>(&sm.qs[P][16 * m + l16][8 * ((4 * d + lg) ^ rsw)]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int a = j == 0 ? a_lo : a_hi;
      if (j == 0 || a_hi != a_lo)
        kb[j][d] = *reinterpret_cast<const bf16x8*>(&sm.ks[P][16 * a + l16][8 * ((4 * d + lg) ^ rsw)]);
    }
  }
  f32x4 gi[2];
  gi[0] = *reinterpret_cast<const f32x4*>(&sm.gt[P][kLgamAt + 16 * a_lo + 4 * lg]);
  gi[1] = *reinterpret_cast<const f32x4*>(&sm.gt[P][kLgamAt + 16 * a_hi + 4 * lg]);
  float gtm[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) gtm[m] = sm.gt[P][kLgamAt + 16 * m + l16];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < 4; ++m) YT[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 acc[2][4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int m = 0; m < 4; ++m) YT[m] = mfma16(sb[d], qa[d][m], YT[m]);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int a = j == 0 ? a_lo : a_hi;
        if ((j == 1 && a_hi == a_lo) || m < a || aqk_owner(a, m) != WS) continue;
        acc[j][m] = mfma16(kb[j][d], qa[d][m], d == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[j][m]);
      }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int a = j == 0 ? a_lo : a_hi;
      if ((j == 1 && a_hi == a_lo) || m < a || aqk_owner(a, m) != WS) continue;
      put_aqk_tile(&sm.frag[P][1][0], a, m, lane, acc[j][m], gtm[m], gi[j]);
    }
}

// Side wave, one chunk: outputs of the chunk (tile of chain wave ws).
template <int P, typename Copy>
__device__ __forceinline__ void side_chunk(SplitSmem& sm, int ws, int lane, float scale,
                                           __amdgpu_buffer_rsrc_t orc, uint32_t ocol, Copy&& copy_next) {
  const int l16 = lane & 15;
  // the copies go first: they then have the whole chunk to land, and Y^T runs
  // while the chain wave is in its VALU-heavy R / Delta phase instead of X
  copy_next();
  f32x4 YT[4];
  switch (ws) {   // uniform
    case 0: side_front<0, P>(sm, lane, YT); break;
    case 1: side_front<1, P>(sm, lane, YT); break;
    case 2: side_front<2, P>(sm, lane, YT); break;
    default: side_front<3, P>(sm, lane, YT); break;
  }
  float sg[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) sg[m] = scale * sm.gt[P][16 * m + l16];
  lds_barrier();   // B2: Delta fragments and every side wave's Aqk tiles visible
  bf16x8 dob[2], fa[2][4];
#pragma unroll
  for (int d = 0; d < 2; ++d) dob[d] = __builtin_bit_cast(bf16x8, sm.dox[ws][d][lane]);
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int d = 0; d < 2; ++d)
      if (!frag_zero(m, d)) fa[d][m] = *reinterpret_cast<const bf16x8*>(&sm.frag[P][1][(frag_slot(m, d) * 64 + lane) * 8]);
  __builtin_amdgcn_sched_barrier(0);
  f32x4 OT[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) OT[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int m = 0; m < 4; ++m)
      if (!frag_zero(m, d)) OT[m] = mfma16(dob[d], fa[d][m], OT[m]);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int t = 16 * m + l16;
    const u32x2 pk = {pack_bf2(sg[m] * YT[m][0] + scale * OT[m][0], sg[m] * YT[m][1] + scale * OT[m][1]),
                      pack_bf2(sg[m] * YT[m][2] + scale * OT[m][2], sg[m] * YT[m][3] + scale * OT[m][3])};
    __builtin_amdgcn_raw_buffer_store_b64(pk, orc, static_cast<uint32_t>(t) * (kVHeads * kDim * 2) + ocol, 0, 0);
  }
}

// Split consumer over the run list: work item = (run, value half, v-head) as
// run * 16 + half * 8 + h.  Runs come longest first.  Work-group wg starts with
// item wg; later items are claimed from a queue (a counter in the list
// header), so a group that finishes early (a short run, an M-run that stopped)
// takes the next longest item.  The claim is issued during the item's last
// chunk, which hides its latency.  A run covers chunks [seg L, min(nch,
// (seg + 1) L)) of its sequence:
//   segment 0           : initial state from `state`, outputs to `out`;
//   B-run, segment >= 1 : zero initial state, outputs O0 to `out`;
//   M-run, segment >= 1 : identity initial state, V = 0, outputs OI to `oi`.
// Final state: new_state for a one-segment sequence, else the segment's slot
// (B-runs and segment 0 in slotb, row-major; M-runs in slotm as the bf16 hi /
// lo MFMA fragments of M^T the scan multiplies with).
__device__ __forceinline__ void split_items(
    SplitSmem& sm, int wg, int nwg, const ListView lv,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ state, float scale, const uint16_t* __restrict__ ws_frag,
    const float* __restrict__ ws_gam,
    uint16_t* __restrict__ out, float* __restrict__ new_state, uint16_t* __restrict__ oi,
    float* __restrict__ slotb, uint16_t* __restrict__ slotm, int* __restrict__ mval, int4* __restrict__ fix,
    int fix_cap) {
  // The run table was written by an earlier launch and is constant here, so
  // it is read through the constant address space: scalar loads, counted in
  // lgkmcnt.  Vector loads would count in vmcnt behind the previous item's
  // final-state stores, and waiting for the descriptor would wait for those.
  const auto* runs_c = (const __attribute__((address_space(4))) u32x4*)lv.runs;
  // First items: when the groups take a whole first wave of 16 runs, the four
  // items of one (run, q/k head) (two v-heads, two halves) go to groups on the
  // same XCD (group id % 8), so the chunk's K / Q rows and both v-heads'
  // fragments are fetched into one L2.  Item (run r, q/k head hq, v-head e of
  // the pair, half) -> group 8 (4 (G / 8) + 2 e + half) + G % 8, G = 4 r + hq.
  // That item's descriptor is requested together with the list header, before
  // the run count says whether the mapping applies (one memory round trip
  // instead of two at the kernel start).  It lies inside the run table either
  // way: nwg is kConsumerGroups only when the table holds at least 16 runs.
  int spec = wg;
  if (nwg == kConsumerGroups) {
    const int x = wg & 7, slot = wg >> 3;
    const int G = 8 * (slot >> 2) + x, k = slot & 3;
    spec = 16 * (G >> 2) + 8 * (k & 1) + kGva * (G & 3) + (k >> 1);
  }
  const u32x4 spec_a = runs_c[2 * (spec >> 4)];
  const u32x4 spec_b = runs_c[2 * (spec >> 4) + 1];
  const auto* hdr_c = (const __attribute__((address_space(4))) int*)lv.hdr;
  const int nruns = hdr_c[0];
  const int seg_len = hdr_c[2];
  // every value is waited for here, so the compiler cannot sink the
  // descriptor loads below the header's wait
  asm volatile("" ::"s"(spec_a), "s"(spec_b), "s"(nruns), "s"(seg_len));
  const auto* gam_c = (const __attribute__((address_space(4))) float*)ws_gam;
  const int nitems = nruns * 2 * kVHeads;
  int* queue = lv.hdr + 8;
  const int first = nitems >= kConsumerGroups ? spec : wg;
  bool use_spec = first == spec;
  constexpr int kFixLane = 4 * 64;   // a side-wave lane appends the M-runs' correction blocks
  // The queue and block counters are bumped by one lane.  An opaque zero
  // offset keeps the compiler from rewriting these atomics into the
  // wave-aggregated form, whose result broadcast waits for the atomic on the
  // spot; the plain atomic is waited for where its result is first used.
  int zero_v;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero_v));
  for (int item = first; item < nitems;) {
  int claimed = 0;   // thread 0: the next item from the queue (once claimed)
  bool has_claim = false;
  auto claim = [&] {
    if (threadIdx.x == 0 && !has_claim) {
      claimed = atomicAdd(queue + zero_v, 1);   // queue position: item nwg + claimed
      has_claim = true;
    }
  };
  const int h = item & 7;
  const int hv = (item >> 3) & 1;
  u32x4 ua = spec_a, ub = spec_b;
  if (!use_spec) {
    ua = runs_c[2 * (item >> 4)];
    ub = runs_c[2 * (item >> 4) + 1];
  }
  use_spec = false;
  const int4 ra = make_int4(static_cast<int>(ua.x), static_cast<int>(ua.y), static_cast<int>(ua.z),
                            static_cast<int>(ua.w));
  const int4 rb = make_int4(static_cast<int>(ub.x), static_cast<int>(ub.y), static_cast<int>(ub.z),
                            static_cast<int>(ub.w));
  const int s = ra.x, slot = ra.z, rfirst = ra.w;
  const bool mrun = (ra.y & kRunM) != 0;
  bool from_state = (ra.y & kRunFromState) != 0;
  const int last_tok = min((ra.y >> 8) & 0xff, kChunk);   // the chunk length indexes 64-entry LDS rows
  const int jseg = ra.y >> 16;
  const long long c0r = static_cast<long long>(static_cast<unsigned>(rb.x)) | (static_cast<long long>(rb.y) << 32);
  const int nrun = rb.w;
  // A warm-up run (kRunWarm) starts `warmup` chunks before its segment: the
  // fewest preceding chunks of the sequence whose map bounds (gate block,
  // written by the prepass) sum below kNegligibleLog2, read newest first, four
  // per round trip; when even all of them do not, it starts at the sequence's
  // first chunk from the initial state.  Every wave computes the same value.
  int warmup = 0;
  if ((ra.y & kRunWarm) != 0 && rb.z > 0) {
    const int before = jseg * seg_len;   // chunks of the sequence before the segment
    float acc = 0.0f;
    while (warmup < before && acc >= kNegligibleLog2) {
      float b4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int back = min(warmup + q + 1, before);
        b4[q] = gam_c[(static_cast<size_t>(rfirst - back) * kVHeads + h) * kGamStride + kBoundAt];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (warmup < before && acc >= kNegligibleLog2) {
          acc += b4[q];
          ++warmup;
        }
      }
    }
    if (acc >= kNegligibleLog2) from_state = true;   // warmup == before: the sequence's initial state
  }
  const int n = rb.z + warmup;   // chunks this item runs, warm-up chunks first
  const int hq = h / kGva;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool chain = w < 4;
  const int wt = w & 3;                          // value tile of this wave pair
  const int lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int vcol = kHalfV * hv + 16 * wt;
  // chunk i of the item is chunk i - warmup of the run (negative: warm-up chunks, all full)
  auto chunk_ref = [&](int i) {
    const int li = i - warmup;
    return ChunkRef{c0r + static_cast<long long>(li) * kChunk, li == nrun - 1 ? last_tok : kChunk, rfirst + li};
  };
  auto kappa = [&](int kt, int rr) { return 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1) + rr; };

  f32x4 st[8];
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (chain) {
    if (mrun) {
#pragma unroll
      for (int kt = 0; kt < 8; ++kt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) st[kt][rr] = kappa(kt, rr) == vcol + l16 ? 1.0f : 0.0f;
    } else if (from_state && state != nullptr) {
      const float* sp = state + ((static_cast<size_t>(s) * kVHeads + h) * kDim + vcol + l16) * kDim;
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) st[kt] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sp + kappa(kt, 0)));
    }
  }
  uint16_t* obase = mrun ? oi : out;
  const uint32_t ocol = 2u * static_cast<uint32_t>(vcol + 4 * lg);
  // output rows of chunk i: none for warm-up chunks (the stores fall outside the resource)
  auto out_rsrc = [&](int i, const ChunkRef& cr) {
    return buf_rsrc(obase + (static_cast<size_t>(cr.c0) * kVHeads + h) * kDim,
                    i < warmup ? 0u : static_cast<uint32_t>(cr.c) * (kVHeads * kDim * 2));
  };
  const SplitDmaLane dl = split_dma_lane(wt, lane, hv);
  // Correction blocks of the segment: chunks [0, formed) get O0 + OI S_j^T in
  // the finish.  Each M-run (once per v-head) reserves a block per chunk with
  // records during its first chunk (the atomic returns before that chunk's
  // closing barrier, with the next chunk's copies), and fills them at its end
  // with blocks of one chunk, or of kFinBlockChunks chunks (see kFinBlockSeg);
  // blocks past `formed` are left empty.  The finish then
  // takes one block per group with a single descriptor load.  The entry
  // repeats the later-segment table's.
  const int fix_max = n;
  int fix_pos = 0;

  // An M-run stops once the bound of its map falls below kNegligibleLog2: its
  // outputs of later chunks are negligible (the correction skips them) and so
  // is its final state.  Every wave accumulates the same bounds in the same
  // order, so the decision is uniform.
  float lbound = 0.0f;
  int formed = n;   // chunks whose outputs were formed
  if (n > 0) {
    if (chain) {
      bf16x8 sb[4];
      state_frags(st, sb);
#pragma unroll
      for (int d = 0; d < 4; ++d) sm.sbx[wt][d][lane] = __builtin_bit_cast(u32x4, sb[d]);
    } else {
      split_dma<0>(sm, chunk_ref(0), dl, wt, h, hq, mrun, q, k, v, ws_frag, ws_gam);
    }
    split_barrier<0>(chain);   // the first chunk's copies and every S fragment in place
    if (mrun && hv == 0 && tid == kFixLane) fix_pos = atomicAdd(lv.hdr + 9 + zero_v, fix_max);
    for (int i = 0; i < n; i += 2) {
      {
        if (i + 1 >= n) claim();
        const ChunkRef cr = chunk_ref(i);
        if (chain) {
          chain_chunk<0>(sm, cr.c, st, wt, lane);
        } else {
          side_chunk<0>(sm, wt, lane, scale, out_rsrc(i, cr), ocol, [&] {
            if (i + 1 < n) split_dma<1>(sm, chunk_ref(i + 1), dl, wt, h, hq, mrun, q, k, v, ws_frag, ws_gam);
          });
        }
        lbound += sm.gt[0][kBoundAt];
        split_barrier<kSideStores>(chain);   // B3: buffer 0 free, buffer 1 landed
      }
      if (mrun && lbound < kNegligibleLog2) {
        formed = i + 1;
        break;
      }
      if (i + 1 < n) {
        if (i + 2 >= n) claim();
        const ChunkRef cr = chunk_ref(i + 1);
        if (chain) {
          chain_chunk<1>(sm, cr.c, st, wt, lane);
        } else {
          side_chunk<1>(sm, wt, lane, scale, out_rsrc(i + 1, cr), ocol, [&] {
            if (i + 2 < n) split_dma<0>(sm, chunk_ref(i + 2), dl, wt, h, hq, mrun, q, k, v, ws_frag, ws_gam);
          });
        }
        lbound += sm.gt[1][kBoundAt];
        split_barrier<kSideStores>(chain);
        if (mrun && lbound < kNegligibleLog2) {
          formed = i + 2;
          break;
        }
      }
    }
  } else {
    lds_barrier();   // every wave has read this item's index before it is replaced
  }
  // The next item is published before the final-state stores: reading the
  // claim's result waits for every earlier vector-memory operation of the
  // wave, and the stores would be among them.
  claim();
  if (threadIdx.x == 0) sm.next_item = nwg + claimed;
  if (mrun && tid == 0) mval[static_cast<size_t>(slot) * kVHeads + h] = formed | (formed < n ? kMNegligible : 0);
  if (mrun && hv == 0 && tid == kFixLane && fix_max > 0) {
    const int4 seg = make_int4(rb.x, rb.y, ((nrun - 1) * kChunk + last_tok) | (jseg << 17), slot - 1);
    const int bsz = formed > kFinBlockChunks && jseg >= kFinBlockSeg ? kFinBlockChunks : 1;
    for (int b = 0; b < fix_max && fix_pos + b < fix_cap; ++b) {
      fix[2 * (fix_pos + b)] = seg;
      fix[2 * (fix_pos + b) + 1] = make_int4(h, b * bsz, min((b + 1) * bsz, formed), 0);
    }
  }

  // a stopped M-run's map is negligible and never read; a warm-up run of a
  // segment before the last keeps no state
  if (chain && slot != kSlotNone && !(mrun && formed < n)) {
    if (slot < 0 || !mrun) {
      float* dst = slot < 0 ? new_state + (static_cast<size_t>(s) * kVHeads + h) * kHeadState
                            : slotb + (static_cast<size_t>(slot) * kVHeads + h) * kHeadState;
      dst += static_cast<size_t>(vcol + l16) * kDim;
      if (slot < 0) {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) __builtin_nontemporal_store(st[kt], reinterpret_cast<f32x4*>(dst + kappa(kt, 0)));
      } else {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) *reinterpret_cast<f32x4*>(dst + kappa(kt, 0)) = st[kt];
      }
    } else {
      // M^T fragments: element (k, k') of M^T goes to fragment (k >> 4, d), lane
      // 16 lg' + (k & 15), slot s with k' = perm_depth(d, lg', s).  This wave
      // holds k' = vcol + l16: d = vcol / 32, lg' = l16 / 4, s = 4 (vcol / 16 & 1) + l16 % 4.
      uint16_t* mb = slotm + (static_cast<size_t>(slot) * kVHeads + h) * kMSlotElems;
      const int d = vcol >> 5;
      const int sidx = 4 * ((vcol >> 4) & 1) + (l16 & 3);
      const int lgp = l16 >> 2;
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int kk = kappa(kt, rr);
          const float x = st[kt][rr];
          const uint16_t hi = f2bf(x);
          const uint16_t lo = f2bf(x - bf2f(hi));
          const size_t e = ((static_cast<size_t>((kk >> 4) * 4 + d) * 2 * 64) + 16 * lgp + (kk & 15)) * 8 + sidx;
          mb[e] = hi;
          mb[e + 512] = lo;
        }
      }
    }
  }
  lds_barrier();   // publishes the next item; the item's stores stay in flight
  item = sm.next_item;
  }
}

// Consumer entry: work-groups [0, g_long) run the split consumer over the
// run list, the rest the full-head consumer over the short-sequence list, so
// both regimes of a mixed batch run concurrently.  Lists come from the plan
// (no host synchronisation); an empty list costs one short round of groups.
union ConsumerLds {
  ConsumerSmem full;
  SplitSmem split;
};

__global__ __launch_bounds__(kSplitThreads)
void consumer_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                     const uint16_t* __restrict__ v, const float* __restrict__ state,
                     int R, int gcap, float scale, int* __restrict__ lists, int num_seqs,
                     int g_long, const uint16_t* __restrict__ ws_frag, const float* __restrict__ ws_gam,
                     uint16_t* __restrict__ out, float* __restrict__ new_state, uint16_t* __restrict__ oi,
                     float* __restrict__ slotb, uint16_t* __restrict__ slotm, int* __restrict__ mval,
                     int4* __restrict__ fix) {
  __shared__ ConsumerLds sm;
  const int bid = blockIdx.x;
  const ListView lv = list_view(lists, num_seqs, gcap);
  if (bid < g_long) {
    split_items(sm.split, bid, g_long, lv, q, k, v, state, scale, ws_frag, ws_gam, out, new_state, oi, slotb,
                slotm, mval, fix, R * kVHeads);
    // an M-run that stopped early may leave its next chunk's copies into LDS in
    // flight: they land before the work-group releases its LDS
    __builtin_amdgcn_s_waitcnt(0);
  } else {
    full_head_items(sm.full, bid - g_long, static_cast<int>(gridDim.x) - g_long, lv.shorts, lv.hdr[1],
                    q, k, v, state, scale, ws_frag, ws_gam, out, new_state);
  }
}

// ============================================================================
// finish: states before segments, output correction, final states
// ============================================================================
// S_{j+1} = S_j M_j + B_j and O_j = O0_j + OI_j S_j^T.  An M-run that stopped
// early (kMNegligible) has a map below 2^-30, so the state after its segment is
// B_j itself: the state before segment j is rebuilt from the latest such
// segment before it (or from S_1), with scan steps only across segments whose
// maps are not negligible.  Work items, one work-group each:
//   a correction block (segment j >= 1, v-head, one or kFinBlockChunks chunks
//        whose OI was formed), as the consumer's M-run appended it: S_j, then
//        out = bf16(O0 + OI S_j^T) for the block's chunks (the other chunks
//        keep O0), chunk by chunk, wave w taking 16-token tile w;
//   (multi-segment sequence, v-head): new_state = S_nseg.
// A scan step forms D = M^T S^T on MFMA with M^T as the M-run stored it (bf16
// hi / lo) and S split into hi / lo from LDS (three products, fp32
// accumulation from B_i).  The correction multiplies OI (bf16) by S as a single
// bf16, as the chunk recurrence does in Q S^T.
constexpr int kFinRow = kDim + 4;   // floats per LDS row of S

union FinishLds {
  float s[kDim][kFinRow];          // S (fp32, row-major, padded)
  u32x4 frag[8][4][64];            // S as correction A fragments: [v-tile][d][lane], slot s = S[16 vt + l16][32 d + 8 lg + s]
};

// One slot state (64 KB, row-major) into registers, thread tid taking the
// 16-byte pieces tid + e * kFinThreads.
constexpr int kFinPer = kDim * kDim / 4 / kFinThreads;
__device__ __forceinline__ void load_slot(const float* __restrict__ src, f32x4 (&t)[kFinPer]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int e = 0; e < kFinPer; ++e) {
    const int q4 = tid + e * kFinThreads;
    t[e] = *reinterpret_cast<const f32x4*>(src + (q4 >> 5) * kDim + (q4 & 31) * 4);
  }
}

// State before segment j of the sequence whose slots start at g0, v-head h,
// into sm.s (fp32).  S_{i+1} is exactly slotb[g0 + i] for i = 0 (S_1) and after
// a negligible map (B_i), so the rebuild starts from the latest such slot.  The
// caller has loaded the usual one: `first` = slotb[g0 + j - 1], `prev` = the
// M-run entry of segment j - 1 (any value with kMNegligible set when j = 1).
__device__ void state_before(FinishLds& sm, int g0, int j, int h, const float* __restrict__ slotb,
                             const uint16_t* __restrict__ slotm, const int* __restrict__ mval, int w, int lane,
                             const f32x4 (&first)[kFinPer], int prev) {
  const int tid = threadIdx.x;
  const int l16 = lane & 15, lg = lane >> 4;
  int i0 = j - 1;
  if ((prev & kMNegligible) == 0) {
    // segment j-1's map is not negligible: step back to the latest slot that is a state
    --i0;
    while (i0 > 0 && (mval[static_cast<size_t>(g0 + i0) * kVHeads + h] & kMNegligible) == 0) --i0;
    f32x4 t[kFinPer];
    load_slot(slotb + (static_cast<size_t>(g0 + i0) * kVHeads + h) * kHeadState, t);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < kFinPer; ++e) {
      const int q4 = tid + e * kFinThreads;
      *reinterpret_cast<f32x4*>(&sm.s[q4 >> 5][(q4 & 31) * 4]) = t[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < kFinPer; ++e) {
      const int q4 = tid + e * kFinThreads;
      *reinterpret_cast<f32x4*>(&sm.s[q4 >> 5][(q4 & 31) * 4]) = first[e];
    }
  }
  __syncthreads();
  for (int i = i0 + 1; i < j; ++i) {
    // wave w forms output k-tiles 2w, 2w+1 for all 128 rows: D = M^T S^T; the
    // step's operand loads are all issued before the first product
    const size_t gh = static_cast<size_t>(g0 + i) * kVHeads + h;
    const uint16_t* mp = slotm + gh * kMSlotElems + lane * 8;
    const float* bp = slotb + gh * kHeadState;
    bf16x8 am[2][4][2];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int hl = 0; hl < 2; ++hl)
          am[e][d][hl] = *reinterpret_cast<const bf16x8*>(mp + (((2 * w + e) * 4 + d) * 2 + hl) * 512);
    f32x4 acc[8][2];
#pragma unroll
    for (int vb = 0; vb < 8; ++vb)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        acc[vb][e] = *reinterpret_cast<const f32x4*>(bp + (16 * vb + l16) * kDim + 16 * (2 * w + e) + 4 * lg);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int vb = 0; vb < 8; ++vb) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        // B fragment: slot s of chunk d is S[16 vb + l16][perm_depth(d, lg, s)]
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(&sm.s[16 * vb + l16][32 * d + 4 * lg]);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(&sm.s[16 * vb + l16][32 * d + 16 + 4 * lg]);
        const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        bf16x8 sh, sl;
        split_frag(x, sh, sl);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          acc[vb][e] = mfma16(am[e][d][0], sh, acc[vb][e]);
          acc[vb][e] = mfma16(am[e][d][0], sl, acc[vb][e]);
          acc[vb][e] = mfma16(am[e][d][1], sh, acc[vb][e]);
        }
      }
    }
    __syncthreads();   // every wave has read S_i
    // acc[vb][e][rr] = S_{i+1}[16 vb + l16][16 (2w + e) + 4 lg + rr]
#pragma unroll
    for (int vb = 0; vb < 8; ++vb)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        *reinterpret_cast<f32x4*>(&sm.s[16 * vb + l16][16 * (2 * w + e) + 4 * lg]) = acc[vb][e];
    __syncthreads();
  }
}

__global__ __launch_bounds__(kFinThreads, 2) void finish_kernel(int* __restrict__ lists, int num_seqs, int gcap,
                                                             const int4* __restrict__ fix, int fix_cap,
                                                             const float* __restrict__ slotb,
                                                             const uint16_t* __restrict__ slotm,
                                                             const int* __restrict__ mval,
                                                             const uint16_t* __restrict__ oi,
                                                             uint16_t* __restrict__ out,
                                                             float* __restrict__ new_state) {
  __shared__ FinishLds sm;
  const ListView lv = list_view(lists, num_seqs, gcap);
  const int nmulti = lv.hdr[3];
  const int ncorr = min(lv.hdr[9], fix_cap);   // correction blocks
  // the blocks were written by the consumer launch: constant here (scalar loads)
  const auto* fix_c = (const __attribute__((address_space(4))) u32x4*)fix;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  // The state items first: they may step through several segment maps.  The
  // grid is one round of groups (two per CU); items past it go out in
  // alternating order, pass k taking group g's item k G + g for even k and
  // (k + 1) G - 1 - g for odd k, so second items land on the groups whose
  // first item was a cheap one (the last correction blocks) rather than on
  // the state items.
  // With a full grid, the group's position in the item order is permuted so
  // that runs of 64 consecutive items (the blocks of one segment and v-head,
  // which load the same segment state and maps) share an XCD (group id % 8)
  // and find those in one L2.
  const int G = static_cast<int>(gridDim.x);
  const int nitem = ncorr + nmulti * kVHeads;
  const int gid = static_cast<int>(blockIdx.x);
  const int slot_g = G == kFinGroups ? 64 * (gid & 7) + (gid >> 3) : gid;
  for (int pass = 0;; ++pass) {
    const int it = (pass & 1) ? (pass + 1) * G - 1 - slot_g : pass * G + slot_g;
    if (it >= nitem) break;
    if (it < nmulti * kVHeads) {
      const int h = it & 7;
      // new_state = S_nseg
      const int4 me = lv.multi[it >> 3];
      // the usual starting slot and the entry that says whether it is the state
      const int jl = me.z;
      const int prev = jl >= 2 ? mval[static_cast<size_t>(me.y + jl - 1) * kVHeads + h] : kMNegligible;
      f32x4 slot0[kFinPer];
      load_slot(slotb + (static_cast<size_t>(me.y + jl - 1) * kVHeads + h) * kHeadState, slot0);
      __syncthreads();   // the previous item's readers of sm are done
      state_before(sm, me.y, jl, h, slotb, slotm, mval, w, lane, slot0, prev);
      float* dst = new_state + (static_cast<size_t>(me.x) * kVHeads + h) * kHeadState;
      for (int e = tid; e < kDim * kDim / 4; e += kFinThreads) {
        const int row = e >> 5, col = (e & 31) * 4;
        *reinterpret_cast<f32x4*>(dst + row * kDim + col) = *reinterpret_cast<const f32x4*>(&sm.s[row][col]);
      }
      continue;
    }
    // block: (first token lo, hi, tokens | j << 17, slot of segment j - 1) and
    // (v-head, first chunk, end chunk): chunks [first, last) need OI S_j^T
    const int item = it - nmulti * kVHeads;
    const u32x4 fa = fix_c[2 * item], fb = fix_c[2 * item + 1];
    const int4 sg = make_int4(static_cast<int>(fa.x), static_cast<int>(fa.y), static_cast<int>(fa.z),
                              static_cast<int>(fa.w));
    const int h = static_cast<int>(fb.x) & 7;
    const int tok = sg.z & ((1 << 17) - 1), j = sg.z >> 17;
    const int g0 = sg.w - (j - 1);
    const int first = static_cast<int>(fb.y);
    const int last = min(static_cast<int>(fb.z), (tok + kChunk - 1) / kChunk);
    if (first >= last) continue;
    // wave w corrects token tile w of each chunk of the block (all 128 value
    // rows); the first chunk's OI and O0 loads are issued before the state is
    // formed, each later chunk's after the previous chunk's stores
    const long long c0s = static_cast<long long>(static_cast<unsigned>(sg.x)) | (static_cast<long long>(sg.y) << 32);
    const uint32_t trow = static_cast<uint32_t>(16 * w + l16) * (kVHeads * kDim * 2);
    bf16x8 b[4];   // [d]: OI rows as B fragments
    u32x2 o0[8];   // [value tile]: O0, four value columns
    __amdgpu_buffer_rsrc_t orc;
    auto load_chunk = [&](int ci) {
      const long long c0 = c0s + static_cast<long long>(ci) * kChunk;
      const int c = min(kChunk, tok - ci * kChunk);
      const size_t rowbase = (static_cast<size_t>(c0) * kVHeads + h) * kDim;
      const uint32_t bytes = static_cast<uint32_t>(c) * (kVHeads * kDim * 2);
      orc = buf_rsrc(out + rowbase, bytes);
      const __amdgpu_buffer_rsrc_t irc = buf_rsrc(oi + rowbase, bytes);
#pragma unroll
      for (int d = 0; d < 4; ++d)
        b[d] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(irc, trow + 2 * (32 * d + 8 * lg), 0, 0));
#pragma unroll
      for (int vt = 0; vt < 8; ++vt) o0[vt] = __builtin_amdgcn_raw_buffer_load_b64(orc, trow + 2 * (16 * vt + 4 * lg), 0, 0);
    };
    // the usual starting slot of the state rebuild, loaded with the outputs
    const int prev = j >= 2 ? mval[static_cast<size_t>(g0 + j - 1) * kVHeads + h] : kMNegligible;
    f32x4 slot0[kFinPer];
    load_slot(slotb + (static_cast<size_t>(g0 + j - 1) * kVHeads + h) * kHeadState, slot0);
    load_chunk(first);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();   // the previous item's readers of sm are done
    state_before(sm, g0, j, h, slotb, slotm, mval, w, lane, slot0, prev);
    // S -> bf16 correction fragments (in place: read, barrier, write)
    u32x4 fr[2][4];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float* sp = &sm.s[16 * (2 * w + e) + l16][32 * d + 8 * lg];
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(sp);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(sp + 4);
        fr[e][d] = u32x4{pack_bf2(x0[0], x0[1]), pack_bf2(x0[2], x0[3]), pack_bf2(x1[0], x1[1]),
                         pack_bf2(x1[2], x1[3])};
      }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int d = 0; d < 4; ++d) sm.frag[2 * w + e][d][lane] = fr[e][d];
    __syncthreads();
    for (int ci = first; ci < last; ++ci) {
      if (ci > first) load_chunk(ci);
#pragma unroll
      for (int vt = 0; vt < 8; ++vt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < 4; ++d) acc = mfma16(__builtin_bit_cast(bf16x8, sm.frag[vt][d][lane]), b[d], acc);
        const u32x2 o = o0[vt];
        const u32x2 o1 = {pack_bf2(bf_lo(o.x) + acc[0], bf_hi(o.x) + acc[1]),
                          pack_bf2(bf_lo(o.y) + acc[2], bf_hi(o.y) + acc[3])};
        __builtin_amdgcn_raw_buffer_store_b64(o1, orc, trow + 2 * (16 * vt + 4 * lg), 0, 0);
      }
    }
  }
}

}  // namespace gdn

extern "C" size_t gdn_prefill_workspace_bytes(int num_seqs, long long total_tokens) {
  if (num_seqs < 0 || total_tokens < 0) return 0;
  return gdn::ws_layout(num_seqs, total_tokens, std::min(gdn::max_segments(total_tokens), gdn::kDefaultSlots)).total;
}

extern "C" size_t gdn_prefill_workspace_min_bytes(int num_seqs, long long total_tokens) {
  if (num_seqs < 0 || total_tokens < 0) return 0;
  return gdn::ws_layout(num_seqs, total_tokens, 0).total;
}

namespace gdn {

// The prefill launches for a workspace of workspace_bytes bytes (both entry
// points below): argument checks first, nothing launched on a rejection.
int prefill_launch(const void* q, const void* k, const void* v, const float* state,
                          const float* A_log, const void* a, const float* dt_bias,
                          const void* b, const void* cu_seqlens, int cu_seqlens_is_int64,
                          int num_seqs, long long total_tokens, float scale, void* output,
                          float* new_state, void* workspace, size_t workspace_bytes, void* stream) {
  if (num_seqs < 0 || total_tokens < 0) return GDN_ERR_INVALID_ARGUMENT;
  if (num_seqs == 0) return GDN_OK;
  if (!cu_seqlens || !new_state || !workspace || !A_log || !dt_bias)
    return GDN_ERR_INVALID_ARGUMENT;
  if (total_tokens > 0 && (!q || !k || !v || !a || !b || !output)) return GDN_ERR_INVALID_ARGUMENT;
  // q, k, v: 16-byte copies straight into LDS; output: 8-byte stores; states:
  // 16-byte accesses; a, b: 2-byte loads; cu_seqlens: 4- or 8-byte loads
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u)
    return GDN_ERR_UNALIGNED;
  if (reinterpret_cast<uintptr_t>(output) & 7u) return GDN_ERR_UNALIGNED;
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 1u) return GDN_ERR_UNALIGNED;
  if (reinterpret_cast<uintptr_t>(cu_seqlens) & (cu_seqlens_is_int64 ? 7u : 3u)) return GDN_ERR_UNALIGNED;
  if ((reinterpret_cast<uintptr_t>(state) | reinterpret_cast<uintptr_t>(new_state)) & 15u)
    return GDN_ERR_UNALIGNED;
  if ((reinterpret_cast<uintptr_t>(A_log) | reinterpret_cast<uintptr_t>(dt_bias)) & 3u) return GDN_ERR_UNALIGNED;
  if (reinterpret_cast<uintptr_t>(workspace) & 255u) return GDN_ERR_UNALIGNED;
  if (state != nullptr && state == new_state) return GDN_ERR_ALIASING;
  const long long R = max_records(num_seqs, total_tokens);
  // every work-item index (records x heads, runs x 16, multi-segment entries x 64) fits an int
  if (R * kVHeads + static_cast<long long>(num_seqs) * kVHeads * 8 > 0x7fffffffLL ||
      max_runs(num_seqs, max_segments(total_tokens)) * 2 * kVHeads > 0x7fffffffLL)
    return GDN_ERR_INVALID_ARGUMENT;
  // as many segment slots as the workspace holds (the planner adapts to them)
  const long long gcap = slots_fitting(num_seqs, total_tokens, workspace_bytes);
  if (gcap < 0) return GDN_ERR_WORKSPACE_TOO_SMALL;
  const WsLayout L = ws_layout(num_seqs, total_tokens, gcap);
  if (!(scale > 0.0f) && !(scale < 0.0f)) scale = 0.08838834764831845f;

  char* ws = static_cast<char*>(workspace);
  auto* frag = reinterpret_cast<uint16_t*>(ws + L.frag_off);
  auto* gam = reinterpret_cast<float*>(ws + L.gam_off);
  auto* rec_start = reinterpret_cast<int*>(ws + L.start_off);
  auto* lists = reinterpret_cast<int*>(ws + L.list_off);
  auto* recs = reinterpret_cast<int4*>(ws + L.rec_off);
  auto* slotb = reinterpret_cast<float*>(ws + L.slotb_off);
  auto* slotm = reinterpret_cast<uint16_t*>(ws + L.slotm_off);
  auto* oi = reinterpret_cast<uint16_t*>(ws + L.oi_off);
  auto* mval = reinterpret_cast<int*>(ws + L.mval_off);
  auto* fix = reinterpret_cast<int4*>(ws + L.fix_off);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  const auto* ab = static_cast<const uint16_t*>(a);
  const auto* bb = static_cast<const uint16_t*>(b);
  auto* ob = static_cast<uint16_t*>(output);
  const int Ri = static_cast<int>(R), gc = static_cast<int>(gcap);

  // at most two chunks in the whole call: one launch, no workspace traffic
  if (total_tokens <= static_cast<long long>(kDirectMaxChunks) * kChunk && num_seqs <= kDirectMaxSeqs) {
    direct_kernel<<<dim3(static_cast<unsigned>(num_seqs * kVHeads)), dim3(kConsumerThreads), 0, st>>>(
        qb, kb, vb, state, A_log, ab, dt_bias, bb, cu_seqlens, cu_seqlens_is_int64, total_tokens, scale, ob,
        new_state);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? GDN_OK : static_cast<int>(e);
  }

  // small batches: every prepass work-group finds its own record (one launch
  // fewer); large ones: a separate plan launch numbers the records once
  const int fused_plan = num_seqs <= kFusedPlanSeqs ? 1 : 0;
  if (!fused_plan)
    plan_kernel<<<dim3(1), dim3(kPlanThreads), 0, st>>>(cu_seqlens, cu_seqlens_is_int64, num_seqs,
                                                        total_tokens, Ri, gc, A_log, dt_bias, rec_start, recs,
                                                        lists);
  // one wave per (record, v-head) while every item fits in one round: two
  // waves per SIMD for up to 2048 items (a lone item's latency matters there),
  // three (a tighter register budget) for up to 3072.  Larger batches take one
  // wave per (record, q/k head): the gram and the K loads are then not
  // repeated per v-head, and up to 512 records start at once.
  const long long items_v = R * kVHeads;
  if (items_v <= kPrepassMaxGroups * kPrepassWaves) {
    const long long g_pre = (items_v + kPrepassWaves - 1) / kPrepassWaves;
    prepass_kernel<false, 2><<<dim3(static_cast<unsigned>(g_pre + fused_plan)), dim3(kPrepassThreads), 0, st>>>(
        kb, A_log, ab, dt_bias, bb, recs, cu_seqlens, cu_seqlens_is_int64, num_seqs, total_tokens,
        Ri, gc, fused_plan, rec_start, lists, frag, gam);
  } else if (items_v <= 3 * (kPrepassMaxGroups / 2) * kPrepassWaves) {
    const long long g_pre = (items_v + kPrepassWaves - 1) / kPrepassWaves;
    prepass_kernel<false, 3><<<dim3(static_cast<unsigned>(g_pre + fused_plan)), dim3(kPrepassThreads), 0, st>>>(
        kb, A_log, ab, dt_bias, bb, recs, cu_seqlens, cu_seqlens_is_int64, num_seqs, total_tokens,
        Ri, gc, fused_plan, rec_start, lists, frag, gam);
  } else {
    const long long g_pre =
        std::min<long long>((R * kQKHeads + kPrepassWaves - 1) / kPrepassWaves, kPrepassMaxGroups);
    prepass_kernel<true, 2><<<dim3(static_cast<unsigned>(g_pre + fused_plan)), dim3(kPrepassThreads), 0, st>>>(
        kb, A_log, ab, dt_bias, bb, recs, cu_seqlens, cu_seqlens_is_int64, num_seqs, total_tokens,
        Ri, gc, fused_plan, rec_start, lists, frag, gam);
  }
  // persistent grids: one work-group per CU per consumer kind at most; a
  // sequence needs 2 chunks (65 tokens) to be long
  const long long g_long =
      total_tokens > kChunk ? std::min<long long>(max_runs(num_seqs, gcap) * 2 * kVHeads, kConsumerGroups) : 0;
  const long long g_short = std::min<long long>(static_cast<long long>(num_seqs) * kVHeads, kConsumerGroups);
  consumer_kernel<<<dim3(static_cast<unsigned>(g_long + g_short)), dim3(kSplitThreads), 0, st>>>(
      qb, kb, vb, state, Ri, gc, scale, lists, num_seqs, static_cast<int>(g_long), frag, gam, ob, new_state, oi,
      slotb, slotm, mval, fix);
  // a second segment needs more than kMinSegChunks chunks in one sequence and a slot
  if (gcap > 0 && total_tokens > static_cast<long long>(kMinSegChunks) * kChunk) {
    const long long g_fin = std::min<long long>(R * kVHeads, kFinGroups);
    finish_kernel<<<dim3(static_cast<unsigned>(g_fin)), dim3(kFinThreads), 0, st>>>(
        lists, num_seqs, gc, fix, static_cast<int>(R * kVHeads), slotb, slotm, mval, oi, ob, new_state);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? GDN_OK : static_cast<int>(err);
}

}  // namespace gdn

extern "C" int gdn_prefill_fwd(const void* q, const void* k, const void* v, const float* state,
                               const float* A_log, const void* a, const float* dt_bias,
                               const void* b, const void* cu_seqlens, int cu_seqlens_is_int64,
                               int num_seqs, long long total_tokens, float scale, void* output,
                               float* new_state, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return gdn::prefill_launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, cu_seqlens_is_int64, num_seqs,
                             total_tokens, scale, output, new_state, workspace, workspace_bytes, stream);
}
