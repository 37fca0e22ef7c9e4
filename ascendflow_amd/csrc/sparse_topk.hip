// Top-k index selection for sparse MLA on gfx950: the step that produces
// cmp_sparse_indices from per-token index scores over compressed positions.
//
// The reference takes cmp_sparse_indices as an input and leaves its producer
// (the top-k indexer) to the caller (docs/operators/sparse-mla.md:8,266). Its
// contract for the tensor is fixed, though: token t of request b may select
// compressed positions in [0, cutoff), cutoff = max(0, C_b R + r_b - n + j + 1)
// / R, at most min(TOPK, C_b, cutoff) of them, ascending, -1 after
// (docs/operators/sparse-mla.md:41-51,79; examples/sparse_attention/attention.py:339-341).
// These kernels take a score per (token, compressed position) and write, for
// every token, the min(TOPK, C_b, cutoff) positions of largest score among
// [0, cutoff), ties to the lower position, in ascending order.
//
// One workgroup per token. The take-th largest score is found by radix
// selection on a monotonic 32-bit key of the score: three digit passes (11,
// 11 and 10 bits from the top), each an LDS histogram over the candidates
// whose key starts with the digits found so far. Then every key above that
// threshold, and the first `need` keys equal to it, are written in position
// order using prefix sums of their counts, so the output is ascending without
// a sort.
//
// Rows of up to 64K positions stay in registers (sparse_topk_resident): the
// row is read once from HBM with 16-byte loads and every pass runs on the
// registers, so the kernel streams the scores at HBM rate. Longer rows use
// sparse_topk_stream, which re-reads the row for each pass.
#include "common.h"
#include "../../include/ascendflow_amd.h"

namespace afa {

constexpr int TK_BINS = 2048;  // widest digit: 11 bits
constexpr int TK_STREAM_THREADS = 256;

// Order-preserving map of a float to an unsigned key: larger float, larger
// key; -0 and +0 share a key; every NaN takes the largest key (NaN ranks
// above +inf, as torch.topk ranks it). No score maps to 0 (the smallest key,
// that of -inf, is 0x007fffff): key 0 marks a position outside the row.
__device__ __forceinline__ uint32_t score_key(float v) {
  const uint32_t b = __float_as_uint(v), mag = b & 0x7fffffffu;
  if (mag > 0x7f800000u) return 0xffffffffu;  // NaN
  if (mag == 0u) return 0x80000000u;          // -0 as +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Exclusive prefix sum over a workgroup of THREADS threads (wave64); the
// total is returned in *total. scratch: THREADS / 64 ints of LDS. Starts with
// a barrier, so scratch may be reused by consecutive calls.
template <int THREADS>
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int up = __shfl_up(incl, d);
    if (lane >= d) incl += up;
  }
  __syncthreads();
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  int before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < THREADS / 64; ++w) {
    const int c = scratch[w];
    before += w < wave ? c : 0;
    sum += c;
  }
  *total = sum;
  return before + incl - v;
}

struct TopkArgs {
  const float* scores;      // [T][C]
  const int32_t* cu;        // [B + 1]
  const int32_t* seq_cmp;   // [B]
  const int32_t* residual;  // [B]
  int32_t* indices;         // [T][1][TOPK]
  int64_t C;                // score columns per token
  int32_t B, T, TOPK, RATIO;
  int32_t vec4;             // rows are 16-byte aligned (C % 4 == 0, aligned base)
};

// Candidates [0, cand) of a token and how many of them it takes, after the
// request lookup: the last b with cu[b] <= token (empty requests have
// cu[b] == cu[b + 1] and are passed over), as gather.py:10-21.
struct TokenBounds {
  int cand, take;
};

__device__ __forceinline__ TokenBounds token_bounds(const TopkArgs& a, int token) {
  int lo = 0, n = a.B;
  while (n > 1) {
    const int half = n >> 1;
    if (a.cu[lo + half] <= token) {
      lo += half;
      n -= half;
    } else {
      n = half;
    }
  }
  const int count_q = a.cu[lo + 1] - a.cu[lo], offset = token - a.cu[lo];
  const int available = a.seq_cmp[lo];
  const int end = available * a.RATIO + a.residual[lo];
  const int cutoff = max(0, end - count_q + offset + 1) / a.RATIO;
  TokenBounds tb;
  tb.cand = (int)min<int64_t>(cutoff, a.C);
  tb.take = min(max(0, min(a.TOPK, min(available, cutoff))), tb.cand);
  return tb;
}

// Writes the -1 tail and the trivial selections; true when nothing is left.
template <int THREADS>
__device__ __forceinline__ bool trivial_selection(const TopkArgs& a, TokenBounds tb, int32_t* out) {
  for (int i = tb.take + (int)threadIdx.x; i < a.TOPK; i += THREADS) out[i] = -1;
  if (tb.take == 0) return true;
  if (tb.take == tb.cand) {  // every candidate is selected
    for (int i = threadIdx.x; i < tb.take; i += THREADS) out[i] = i;
    return true;
  }
  return false;
}

// One digit of the radix selection, after hist[0, bins) holds the counts of
// the remaining keys: finds the bin holding the need-th largest remaining key
// and returns it, with *above = the count in the bins above it. Ends with a
// barrier, so hist may be cleared next.
template <int THREADS>
__device__ __forceinline__ int choose_bin(const int* hist, int bins, int need, int* scan_scratch, int* choice,
                                          int* above) {
  const int per = bins / THREADS, tid = threadIdx.x;  // thread t sums bins from the top
  int local = 0;
  for (int q = 0; q < per; ++q) local += hist[bins - 1 - (tid * per + q)];
  int total = 0;
  const int before = block_exclusive_scan<THREADS>(local, scan_scratch, &total);
  if (before < need && before + local >= need) {
    int acc = before;
    for (int q = 0; q < per; ++q) {
      const int bin = bins - 1 - (tid * per + q);
      const int c = hist[bin];
      if (acc + c >= need) {
        choice[0] = bin;
        choice[1] = acc;
        break;
      }
      acc += c;
    }
  }
  __syncthreads();
  const int bin = choice[0];
  *above = choice[1];
  __syncthreads();
  return bin;
}

constexpr int DIGIT_SHIFT[3] = {21, 10, 0};
constexpr int DIGIT_WIDTH[3] = {11, 11, 10};

// Resident form: THREADS threads, each holding V4 groups of 4 consecutive
// positions (group v of thread t covers [(v THREADS + t) 4, +4)), so a row of
// up to THREADS V4 4 positions is read once, with coalesced 16-byte loads.
template <int THREADS, int V4>
__global__ __launch_bounds__(THREADS) void sparse_topk_resident(TopkArgs a) {
  constexpr int WAVES = THREADS / 64, N = V4 * 4;
  static_assert(V4 * WAVES <= THREADS, "the chunk table is scanned by one pass of the workgroup");
  __shared__ int hist[TK_BINS];
  __shared__ int scan_scratch[WAVES];
  __shared__ int choice[2];
  __shared__ int table_gt[V4 * WAVES], table_eq[V4 * WAVES];
  const int token = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const TokenBounds tb = token_bounds(a, token);
  int32_t* out = a.indices + (size_t)token * a.TOPK;
  if (trivial_selection<THREADS>(a, tb, out)) return;
  const float* row = a.scores + (size_t)token * a.C;

  uint32_t key[N];
#pragma unroll
  for (int v = 0; v < V4; ++v) {
    const int i0 = (v * THREADS + tid) * 4;
    if (a.vec4) {
      // i0 < cand <= C with C % 4 == 0: the whole group lies inside the row.
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i0 < tb.cand) f = *reinterpret_cast<const float4*>(row + i0);
      key[4 * v + 0] = i0 + 0 < tb.cand ? score_key(f.x) : 0u;
      key[4 * v + 1] = i0 + 1 < tb.cand ? score_key(f.y) : 0u;
      key[4 * v + 2] = i0 + 2 < tb.cand ? score_key(f.z) : 0u;
      key[4 * v + 3] = i0 + 3 < tb.cand ? score_key(f.w) : 0u;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) key[4 * v + e] = i0 + e < tb.cand ? score_key(row[i0 + e]) : 0u;
    }
  }

  uint32_t prefix = 0, prefix_mask = 0;
  int need = tb.take;
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = DIGIT_SHIFT[pass], bins = 1 << DIGIT_WIDTH[pass];
    for (int i = tid; i < bins; i += THREADS) hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const uint32_t k = key[j];
      if (k != 0u && (k & prefix_mask) == prefix) atomicAdd(&hist[(k >> shift) & (uint32_t)(bins - 1)], 1);
    }
    __syncthreads();
    int above = 0;
    const int digit = choose_bin<THREADS>(hist, bins, need, scan_scratch, choice, &above);
    need -= above;
    prefix |= (uint32_t)digit << shift;
    prefix_mask |= (uint32_t)(bins - 1) << shift;
  }

  // Output slot of a selected key = keys above the threshold before it in
  // position order + min(equal keys before it, need). Position order is
  // (group, wave, lane, element): counts per (group, wave) go through one
  // table scan. A wave holds at most 256 keys of each kind, so the wave scans
  // carry both counts in one word (equal << 16 | above).
  const uint32_t threshold = prefix;
  int packed_incl[V4];
#pragma unroll
  for (int v = 0; v < V4; ++v) {
    int packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t k = key[4 * v + e];
      packed += k > threshold ? 1 : (k == threshold ? 0x10000 : 0);
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int up = __shfl_up(packed, d);
      if (lane >= d) packed += up;
    }
    packed_incl[v] = packed;
    if (lane == 63) {
      table_gt[v * WAVES + wave] = packed & 0xffff;
      table_eq[v * WAVES + wave] = packed >> 16;
    }
  }
  __syncthreads();
  {
    constexpr int ENTRIES = V4 * WAVES;
    const int g = tid < ENTRIES ? table_gt[tid] : 0, q = tid < ENTRIES ? table_eq[tid] : 0;
    int total = 0;
    const int g_before = block_exclusive_scan<THREADS>(g, scan_scratch, &total);
    const int q_before = block_exclusive_scan<THREADS>(q, scan_scratch, &total);
    if (tid < ENTRIES) {  // every read of the table happened before the scans' barriers
      table_gt[tid] = g_before;
      table_eq[tid] = q_before;
    }
  }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < V4; ++v) {
    int own = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t k = key[4 * v + e];
      own += k > threshold ? 1 : (k == threshold ? 0x10000 : 0);
    }
    if (own == 0) continue;
    int gt_before = table_gt[v * WAVES + wave] + (packed_incl[v] & 0xffff) - (own & 0xffff);
    int eq_before = table_eq[v * WAVES + wave] + (packed_incl[v] >> 16) - (own >> 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t k = key[4 * v + e];
      const int position = (v * THREADS + tid) * 4 + e;
      if (k > threshold) {
        const int at = gt_before + min(eq_before, need);
        if (at < tb.take) out[at] = position;
        ++gt_before;
      } else if (k == threshold) {
        if (eq_before < need && gt_before + eq_before < tb.take) out[gt_before + eq_before] = position;
        ++eq_before;
      }
    }
  }
}

// Streaming form, for rows of any length: every pass re-reads the row.
__global__ __launch_bounds__(TK_STREAM_THREADS) void sparse_topk_stream(TopkArgs a) {
  constexpr int THREADS = TK_STREAM_THREADS;
  __shared__ int hist[TK_BINS];
  __shared__ int scan_scratch[THREADS / 64];
  __shared__ int choice[2];
  const int token = blockIdx.x, tid = threadIdx.x;
  const TokenBounds tb = token_bounds(a, token);
  int32_t* out = a.indices + (size_t)token * a.TOPK;
  if (trivial_selection<THREADS>(a, tb, out)) return;
  const float* row = a.scores + (size_t)token * a.C;
  const int cand = tb.cand;

  uint32_t prefix = 0, prefix_mask = 0;
  int need = tb.take;
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = DIGIT_SHIFT[pass], bins = 1 << DIGIT_WIDTH[pass];
    for (int i = tid; i < bins; i += THREADS) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < cand; i += THREADS) {
      const uint32_t k = score_key(row[i]);
      if ((k & prefix_mask) == prefix) atomicAdd(&hist[(k >> shift) & (uint32_t)(bins - 1)], 1);
    }
    __syncthreads();
    int above = 0;
    const int digit = choose_bin<THREADS>(hist, bins, need, scan_scratch, choice, &above);
    need -= above;
    prefix |= (uint32_t)digit << shift;
    prefix_mask |= (uint32_t)(bins - 1) << shift;
  }

  // Chunks of THREADS positions in order; one scan per chunk counts both
  // kinds (equal keys in the high half-word, larger keys in the low one).
  const uint32_t threshold = prefix;
  int written = 0, equal_seen = 0;
  for (int base = 0; base < cand; base += THREADS) {
    const int i = base + tid;
    const uint32_t k = i < cand ? score_key(row[i]) : 0u;
    const bool gt = k > threshold, eq = k == threshold;  // k == 0 past the row
    int both = 0;
    const int before = block_exclusive_scan<THREADS>((eq ? 0x10000 : 0) | (gt ? 1 : 0), scan_scratch, &both);
    const int eq_left = max(0, need - equal_seen);  // equal keys still to take
    const int eq_before = before >> 16;
    const int at = written + (before & 0xffff) + min(eq_before, eq_left);
    if ((gt || (eq && eq_before < eq_left)) && at < tb.take) out[at] = i;
    written += (both & 0xffff) + min(both >> 16, eq_left);
    equal_seen += both >> 16;
    if (written >= tb.take) break;  // uniform: every thread sees the same totals
  }
}

template <int THREADS, int V4>
static void launch_resident(const TopkArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((sparse_topk_resident<THREADS, V4>), dim3((unsigned)a.T), dim3(THREADS), 0, stream, a);
}

}  // namespace afa

using namespace afa;

extern "C" int launch_sparse_topk_indices(void* stream, const float* scores, const int32_t* cu_seqlens_q,
                                          const int32_t* seqused_cmp_kv, const int32_t* cmp_residual_kv,
                                          int32_t* cmp_sparse_indices, const SparseTopkParams* params) {
  if (!params) return AFA_E_NULL;
  if (params->B <= 0 || params->T <= 0 || params->TOPK <= 0 || params->C <= 0) return AFA_E_SHAPE;
  if (params->RATIO != 1 && params->RATIO != 2) return AFA_E_SHAPE;
  if (params->C > 0x7fffffffLL) return AFA_E_SHAPE;
  if (!scores || !cu_seqlens_q || !seqused_cmp_kv || !cmp_residual_kv || !cmp_sparse_indices) return AFA_E_NULL;
  TopkArgs a;
  a.scores = scores;
  a.cu = cu_seqlens_q;
  a.seq_cmp = seqused_cmp_kv;
  a.residual = cmp_residual_kv;
  a.indices = cmp_sparse_indices;
  a.C = params->C;
  a.B = params->B;
  a.T = params->T;
  a.TOPK = params->TOPK;
  a.RATIO = params->RATIO;
  a.vec4 = (params->C % 4 == 0) && (reinterpret_cast<uintptr_t>(scores) % 16 == 0);
  hipStream_t s = (hipStream_t)stream;
  // Resident capacity THREADS * V4 * 4 positions; the smallest form that holds
  // a full row (no token has more than C candidates).
  if (a.C <= 4096)
    launch_resident<256, 4>(a, s);
  else if (a.C <= 16384)
    launch_resident<512, 8>(a, s);
  else if (a.C <= 65536)
    launch_resident<1024, 16>(a, s);
  else
    hipLaunchKernelGGL(sparse_topk_stream, dim3((unsigned)a.T), dim3(TK_STREAM_THREADS), 0, s, a);
  return (int)hipGetLastError();
}
