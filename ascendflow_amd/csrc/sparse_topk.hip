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
// One workgroup per token; the selection works on a monotonic 32-bit key of
// each score. sparse_topk_filter (rows up to 256K positions; 256 threads up
// to 32K positions, 1024 beyond):
//   1. sample: four keys per thread (two in the 1024-thread form: 2048
//      keys), in blocks of 16 consecutive positions
//      evenly spaced over the row (issued with the request lookup, over the
//      whole allocated row, and kept when the token's candidates cover at
//      least half of it; shorter rows are sampled again over their
//      candidates); a two-digit radix selection on the sample (the top 22
//      bits of the key: an estimate needs no more) gives an estimate of the
//      threshold, taken at 1.25x the expected rank plus 8 (256 threads) or
//      twice it plus 16 (1024), so that somewhat more than `take` keys reach
//      it;
//   2. filter: one streaming pass over the row (16-byte loads, several in
//      flight per thread) appends every key >= estimate, with its position,
//      to an LDS buffer (wave ballots, one LDS atomic per wave and step);
//   3. exact selection: radix selection (digits of 11, 11 and 10 bits, LDS
//      histograms) over the buffer, giving the threshold key and how many keys
//      equal to it are taken; if fewer than `take` keys reached the estimate,
//      or the buffer overflowed, the row is filtered again at another sample
//      rank (binary search, up to four passes), and failing that the same
//      selection runs over the whole row, re-reading it per digit (same
//      result, slower);
//   4. output: keys above the threshold, and keys equal to it, set bits in two
//      LDS bitmaps over the row's positions; one scan of the bitmaps writes
//      the positions in ascending order, taking the first `need` equal keys.
// The row is read once from HBM on the common path. sparse_topk_stream
// serves longer rows: every digit, and the output, re-read the row.
#include <algorithm>

#include "common.h"
#include "../../include/ascendflow_amd.h"

namespace afa {

constexpr int TK_BINS = 2048;  // widest digit: 11 bits
constexpr int TK_UNROLL = 4;    // 4-position groups in flight per thread in a streaming pass
constexpr int TK_FILTER_ROUNDS = 4;  // filter passes before the whole-row selection
// Sample keys per thread for the threshold estimate: 4 x 256 = 1024 keys in
// the 256-thread form, whose buffer of 2 TOPK entries needs the closer
// estimate; 2 x 1024 = 2048 in the 1024-thread form (4096 entries), where
// the sample's histogram atomics, crowded into the few bins that the leading
// digit of similar scores falls into, had made the estimate a tenth of the
// kernel (decode 38.4 -> 36.3 µs against 4096 keys).
template <int THREADS> constexpr int TK_SAMPLES = THREADS <= 256 ? 4 : 2;
constexpr int TK_WIDE_CAP = 4096;    // filter buffer entries of the 1024-thread form
constexpr int64_t TK_FILTER_MAX_C = 262144;  // two LDS bitmaps of C bits each
// Word 3 of a raw buffer resource on gfx9-family GPUs (32-bit data format,
// no swizzle): with stride 0, a load at byte offset >= num_records returns 0.
constexpr int BUFFER_WORD3 = 0x00020000;
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

struct TopkArgs {
  const float* scores;      // [T][C]
  const int32_t* cu;        // [B + 1]
  const int32_t* seq_cmp;   // [B]
  const int32_t* residual;  // [B]
  int32_t* indices;         // [T][1][TOPK]
  int64_t C;                // score columns per token
  int32_t B, T, TOPK, RATIO;
  int32_t cap;              // filter buffer entries (dynamic LDS)
  int32_t words;            // bitmap words per row in dynamic LDS: ceil(C / 32)
};

// Candidates [0, cand) of a token and how many of them it takes, after the
// request lookup: the last b with cu[b] <= token (empty requests have
// cu[b] == cu[b + 1] and are passed over), as gather.py:10-21.
struct TokenBounds {
  int cand, take;
};

// Bounds of a token of the request holding cu[b] = begin, cu[b + 1] = next,
// seq_cmp[b] = available, residual[b] = residual.
__device__ __forceinline__ TokenBounds bounds_of(const TopkArgs& a, int token, int begin, int next, int available,
                                                 int residual) {
  const int count_q = next - begin, offset = token - begin;
  const int end = available * a.RATIO + residual;
  const int cutoff = max(0, end - count_q + offset + 1) / a.RATIO;
  TokenBounds tb;
  tb.cand = (int)min<int64_t>(cutoff, a.C);
  tb.take = min(max(0, min(a.TOPK, min(available, cutoff))), tb.cand);
  return tb;
}

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
  return bounds_of(a, token, a.cu[lo], a.cu[lo + 1], a.seq_cmp[lo], a.residual[lo]);
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

// Exclusive prefix sums of two values over the workgroup, sharing barriers;
// totals in total[0..1]. scratch: 2 THREADS / 64 ints of LDS.
template <int THREADS>
__device__ __forceinline__ void block_exclusive_scan2(int& a, int& b, int* scratch, int* total) {
  constexpr int WAVES = THREADS / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ia = wave_inclusive_scan(a), ib = wave_inclusive_scan(b);
  __syncthreads();
  if (lane == 63) {
    scratch[wave] = ia;
    scratch[WAVES + wave] = ib;
  }
  __syncthreads();
  int before_a = 0, before_b = 0, sum_a = 0, sum_b = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    const int ca = scratch[w], cb = scratch[WAVES + w];
    before_a += w < wave ? ca : 0;
    before_b += w < wave ? cb : 0;
    sum_a += ca;
    sum_b += cb;
  }
  total[0] = sum_a;
  total[1] = sum_b;
  a = before_a + ia - a;
  b = before_b + ib - b;
}

constexpr int DIGIT_SHIFT[3] = {21, 10, 0};
constexpr int DIGIT_WIDTH[3] = {11, 11, 10};

// LDS of the radix selections: two histograms, used alternately, so the one
// for the next digit is cleared while a digit is chosen from the other.
// PACKED: 16-bit counts, two bins per word, for selections over fewer than
// 2^16 keys (a count never carries into its neighbour).
template <bool PACKED>
struct RadixLds {
  static constexpr int WORDS = PACKED ? TK_BINS / 2 : TK_BINS;
  alignas(16) uint32_t hist[2][WORDS];
  int choice[2];  // bin of the digit, keys in the bins above it
  __device__ __forceinline__ void add(int parity, int bin, int n) {
    if constexpr (PACKED)
      atomicAdd(&hist[parity][bin >> 1], (uint32_t)n << ((bin & 1) * 16));
    else
      atomicAdd(&hist[parity][bin], (uint32_t)n);
  }
  __device__ __forceinline__ int get(int parity, int bin) const {
    if constexpr (PACKED)
      return (int)((hist[parity][bin >> 1] >> ((bin & 1) * 16)) & 0xffffu);
    else
      return (int)hist[parity][bin];
  }
};

// Radix selection of the rank-th largest key among those a key source
// yields: for_each_key(f) calls f(key) for every key of the source held by
// this thread. Returns that key, with *need_out = how many keys equal to it
// are among the rank largest; with PASSES < 3 digits, the key's leading
// DIGIT_SHIFT[PASSES - 1] bits (the rest zero) and the count for that prefix.
// Per digit: LDS histogram atomics, one barrier, wave 0 finds the digit's bin
// (a scan over lanes from the top bin) while the other waves clear the other
// histogram, one barrier. Expects hist[parity] cleared and leaves
// hist[parity] (flipped) cleared.
template <int THREADS, bool PACKED, int PASSES = 3, typename ForEachKey>
__device__ __forceinline__ uint32_t radix_select(ForEachKey for_each_key, int rank, RadixLds<PACKED>& lds, int& parity,
                                                 int* need_out) {
  static_assert(PASSES >= 1 && PASSES <= 3, "one to three digits");
  static_assert(THREADS > 64, "the histogram is cleared by the waves other than wave 0");
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t prefix = 0, prefix_mask = 0;
  int need = rank;
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    const int shift = DIGIT_SHIFT[pass], bins = 1 << DIGIT_WIDTH[pass];
    const int cur = parity;
    for_each_key([&](uint32_t k) {
      // Lanes whose key falls in the same bin as the first counting lane's add
      // together in one atomic (keys often share their leading digit); the
      // others add their own.
      const bool counts = (k & prefix_mask) == prefix;
      const uint64_t active = __ballot(counts);
      if (active == 0) return;  // uniform
      const int bin = (int)((k >> shift) & (uint32_t)(bins - 1));
      const int leader = (int)__builtin_ctzll(active);
      const int lead_bin = __builtin_amdgcn_readlane(bin, leader);  // leader is wave-uniform
      const uint64_t same = __ballot(counts && bin == lead_bin);
      if (lane == leader) lds.add(cur, lead_bin, __popcll(same));
      else if (counts && bin != lead_bin) lds.add(cur, bin, 1);
    });
    __syncthreads();
    if (tid < 64) {
      // Lane l sums bins [bins - (l + 1) per, bins - l per): U = 2, 4 or 8
      // aligned 16-byte units of whole words, read in the order c, c + 1, ...
      // (mod U) with c chosen so that the 16 lanes one ds_read_b128 pass
      // serves (four quads whose (lane >> 3) & 3 differ) touch 16 distinct
      // bank groups. Packed words are summed whole: no half-word sum reaches
      // 2^16. The lane whose bins hold the need-th key is found by a scan over
      // the lanes, then its bins are read one per lane and scanned the same way.
      const int per = bins / 64;
      const int W = PACKED ? per / 2 : per, U = W / 4;
      const int quad = (lane >> 3) & 3;
      const int c = U == 2 ? (quad & 1) : U == 4 ? quad : (((lane >> 1) & 1) | (quad << 1));
      const uint32_t* words = lds.hist[cur] + (bins - (lane + 1) * per) / (PACKED ? 2 : 1);
      uint32_t sum = 0;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        if (it < U) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(words + 4 * ((c + it) & (U - 1)));
          sum += (v[0] + v[1]) + (v[2] + v[3]);
        }
      }
      const int local = PACKED ? (int)((sum & 0xffffu) + (sum >> 16)) : (int)sum;
      const int incl = wave_inclusive_scan(local);
      const int owner = (int)__builtin_ctzll(__ballot(incl - local < need && incl >= need));
      const int above = __builtin_amdgcn_readlane(incl - local, owner);  // owner is wave-uniform
      const int count = lane < per ? lds.get(cur, bins - 1 - (owner * per + lane)) : 0;
      const int incl2 = wave_inclusive_scan(count);
      const int q = (int)__builtin_ctzll(__ballot(lane < per && above + incl2 >= need));
      if (lane == q) {
        lds.choice[0] = bins - 1 - (owner * per + q);
        lds.choice[1] = above + incl2 - count;
      }
    } else {
      uint32_t* spare = lds.hist[parity ^ 1];
      for (int i = 4 * (tid - 64); i < RadixLds<PACKED>::WORDS; i += 4 * (THREADS - 64))
        *reinterpret_cast<u32x4*>(spare + i) = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    need -= lds.choice[1];
    prefix |= (uint32_t)lds.choice[0] << shift;
    prefix_mask |= (uint32_t)(bins - 1) << shift;
    parity ^= 1;
  }
  *need_out = need;
  return prefix;
}

// One streaming pass over the candidates [0, cand) of a row read through a
// buffer resource of range cand * 4 bytes (loads past it return zeros without
// touching memory): f(key, position) is called by every thread of the wave
// together, TK_UNROLL * 4 times per step, with key 0 for a position past the
// candidates (no score maps to key 0). VEC: 16-byte loads of 4 consecutive
// positions (rows 16-byte aligned); otherwise 4-byte loads.
template <int THREADS, bool VEC>
__device__ __forceinline__ int stream_position(int base, int j) {
  const int tid = threadIdx.x;
  return VEC ? base + ((j >> 2) * THREADS + tid) * 4 + (j & 3) : base + j * THREADS + tid;
}

// The same pass handing each step's UNROLL * 4 keys to f at once:
// f(keys, base), keys[j] being the key of position stream_position(base, j).
template <int THREADS, bool VEC, int UNROLL, typename F>
__device__ __forceinline__ void stream_row_steps(__amdgpu_buffer_rsrc_t rsrc, int cand, F f) {
  constexpr int STEP = THREADS * 4 * UNROLL;
  for (int base = 0; base < cand; base += STEP) {
    uint32_t w[UNROLL * 4];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if constexpr (VEC) {
        const u32x4 x = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, stream_position<THREADS, VEC>(base, 4 * u) * 4, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * u + e] = x[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[4 * u + e] =
              __builtin_amdgcn_raw_buffer_load_b32(rsrc, stream_position<THREADS, VEC>(base, 4 * u + e) * 4, 0, 0);
      }
    }
    uint32_t keys[UNROLL * 4];
#pragma unroll
    for (int j = 0; j < UNROLL * 4; ++j)
      keys[j] = stream_position<THREADS, VEC>(base, j) < cand ? score_key(__uint_as_float(w[j])) : 0u;
    f(keys, base);
  }
}

template <int THREADS, bool VEC, typename F>
__device__ __forceinline__ void stream_row(__amdgpu_buffer_rsrc_t rsrc, int cand, F f) {
  constexpr int STEP = THREADS * 4 * TK_UNROLL;
  for (int base = 0; base < cand; base += STEP) {
    uint32_t w[TK_UNROLL * 4];
#pragma unroll
    for (int u = 0; u < TK_UNROLL; ++u) {
      if constexpr (VEC) {
        const u32x4 x = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, stream_position<THREADS, VEC>(base, 4 * u) * 4, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * u + e] = x[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[4 * u + e] =
              __builtin_amdgcn_raw_buffer_load_b32(rsrc, stream_position<THREADS, VEC>(base, 4 * u + e) * 4, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < TK_UNROLL * 4; ++j) {
      const int p = stream_position<THREADS, VEC>(base, j);
      f(p < cand ? score_key(__uint_as_float(w[j])) : 0u, p);
    }
  }
}

__device__ __forceinline__ int lane_rank(uint64_t mask) {  // set bits of mask below this lane
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

template <bool COMPACT> struct BufferPosition { typedef int type; };
template <> struct BufferPosition<true> { typedef uint16_t type; };

// COMPACT (rows up to 32K positions, 256 threads): 16-bit histogram counts
// and buffer positions, so that more workgroups fit in a CU's LDS.
// Eight waves per SIMD (at most 64 VGPRs): two 1024-thread or eight 256-thread
// workgroups per CU, as many as the LDS holds.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS, 8) void sparse_topk_filter(TopkArgs a) {
  constexpr bool COMPACT = THREADS <= 256;
  // 4-position groups per thread and step of the filter pass.
  constexpr int FILTER_UNROLL = THREADS <= 256 ? TK_UNROLL : TK_UNROLL / 2;
  typedef typename BufferPosition<COMPACT>::type Position;
  // Dynamic LDS: two bitmaps of a.words words (keys above the threshold, keys
  // equal to it), then (COMPACT) the buffer of a.cap keys and positions; the
  // 1024-thread form keeps a static buffer of TK_WIDE_CAP entries.
  extern __shared__ uint32_t dynamic_lds[];
  __shared__ uint32_t wide_key[COMPACT ? 1 : TK_WIDE_CAP];
  __shared__ int wide_pos[COMPACT ? 1 : TK_WIDE_CAP];
  const int CAP = COMPACT ? a.cap : TK_WIDE_CAP;
  uint32_t* const bitmaps = dynamic_lds;
  uint32_t* const buf_key = COMPACT ? dynamic_lds + 2 * a.words : wide_key;
  Position* const buf_pos =
      COMPACT ? reinterpret_cast<Position*>(dynamic_lds + 2 * a.words + a.cap) : reinterpret_cast<Position*>(wide_pos);
  __shared__ RadixLds<COMPACT> radix;
  __shared__ int scan_scratch[2 * THREADS / 64];
  __shared__ int reached;
  __shared__ int request_lds[4];
  constexpr int WAVES = THREADS / 64;
  const int token = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // 1. Sample: S keys in blocks of 16 consecutive positions (64 bytes), the
  // S / 16 blocks evenly spaced over a range of n positions (block b from
  // position floor(b n / (S / 16))), so the sample touches few cache lines;
  // thread t holds samples SPT t .. SPT t + SPT - 1. The first sample, S =
  // min(SPT THREADS, C) over the whole allocated row (n = C), goes out before
  // the request lookup; its keys at positions past the token's candidates are
  // left out, and when the candidates cover less than half of the row (or C
  // < SPT THREADS) the row is sampled again over them (n = cand,
  // S = min(SPT THREADS, cand), a row shorter than that whole).
  // A sample shorter than SPT THREADS is the whole range (block
  // positions i); otherwise it has SAMPLE_BLOCKS blocks, a power of two, so
  // floor(b n / SAMPLE_BLOCKS) is a shift. The loads are unconditional
  // (positions past the buffer's range read 0) and their words are turned
  // into keys only where they are used, so that the four go out together
  // with the request lookup's and share its round trip.
  constexpr int SPT = TK_SAMPLES<THREADS>;
  constexpr int SAMPLE_BLOCKS = SPT * THREADS / 16;
  constexpr int SAMPLE_SHIFT = __builtin_ctz(SAMPLE_BLOCKS);
  static_assert((SAMPLE_BLOCKS & (SAMPLE_BLOCKS - 1)) == 0, "sample blocks must be a power of two");
  auto sample_position = [&](int i, int64_t n, int s) {
    return s < SPT * THREADS ? i : (int)(((int64_t)(i >> 4) * n) >> SAMPLE_SHIFT) + (i & 15);
  };
  const int samples_c = (int)min<int64_t>(SPT * THREADS, a.C);
  const __amdgpu_buffer_rsrc_t rsrc_row = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.scores + (size_t)token * a.C), (short)0, (int)(a.C * 4), BUFFER_WORD3);
  uint32_t sample[SPT];  // the score words, then their keys
  int sample_pos[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    sample_pos[j] = sample_position(tid * SPT + j, a.C, samples_c);
    sample[j] = __builtin_amdgcn_raw_buffer_load_b32(rsrc_row, sample_pos[j] * 4, 0, 0);
  }
  // Request lookup. B <= THREADS: one round trip, thread b loading request
  // b's cu[b], cu[b + 1], seq_cmp[b] and residual[b]; the token's request is
  // #{b: cu[b] <= token} - 1 (as in token_bounds), whose thread hands its
  // values to the others through LDS. Larger B: the binary search.
  TokenBounds tb;
  if (a.B <= THREADS) {
    int begin = 0, next = 0, available = 0, residual = 0;
    if (tid < a.B) {
      begin = a.cu[tid];
      next = a.cu[tid + 1];
      available = a.seq_cmp[tid];
      residual = a.residual[tid];
    }
    const int below = __popcll(__ballot(tid < a.B && begin <= token));
    if (lane == 0) scan_scratch[wave] = below;
    __syncthreads();
    int requests = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) requests += scan_scratch[w];
    if (tid == max(requests - 1, 0)) {  // request 0 at least (cu[0] = 0 <= token)
      request_lds[0] = begin;
      request_lds[1] = next;
      request_lds[2] = available;
      request_lds[3] = residual;
    }
    __syncthreads();
    tb = bounds_of(a, token, request_lds[0], request_lds[1], request_lds[2], request_lds[3]);
  } else {
    tb = token_bounds(a, token);
  }
  int32_t* out = a.indices + (size_t)token * a.TOPK;
  if (trivial_selection<THREADS>(a, tb, out)) return;
  const int cand = tb.cand, take = tb.take, words = (cand + 31) >> 5;
  uint32_t* above_bits = bitmaps;
  uint32_t* equal_bits = bitmaps + words;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.scores + (size_t)token * a.C), (short)0, cand * 4, BUFFER_WORD3);
  const bool whole_row_sample = samples_c == SPT * THREADS && 2 * (int64_t)cand >= a.C;  // uniform
  int samples = 0;           // keys in the sample
  uint32_t sample_mask = 0;  // bit j: sample[j] is one of them
  if (whole_row_sample) {
    int mine = 0;
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      sample[j] = score_key(__uint_as_float(sample[j]));  // every sample is in [0, C) here
      const bool in_row = sample_pos[j] < cand;
      sample_mask |= in_row ? 1u << j : 0u;
      mine += in_row ? 1 : 0;
    }
    mine = __builtin_amdgcn_readlane(wave_inclusive_scan(mine), 63);
    if (lane == 0) scan_scratch[WAVES + wave] = mine;  // summed after the barrier below
  } else {
    samples = min(SPT * THREADS, cand);
#pragma unroll
    for (int j = 0; j < SPT; ++j)
      sample[j] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, sample_position(tid * SPT + j, cand, samples) * 4, 0, 0);
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const int i = tid * SPT + j;
      sample[j] = i < samples ? score_key(__uint_as_float(sample[j])) : 0u;
      sample_mask |= i < samples ? 1u << j : 0u;
    }
  }
  for (int i = tid; i < 2 * words; i += THREADS) bitmaps[i] = 0u;
  for (int i = tid; i < RadixLds<COMPACT>::WORDS; i += THREADS) radix.hist[0][i] = 0u;
  if (tid == 0) reached = 0;
  __syncthreads();
  if (whole_row_sample) {
#pragma unroll
    for (int w = 0; w < WAVES; ++w) samples += scan_scratch[WAVES + w];
  }
  int parity = 0, unused = 0;

  // 2. Filter: keys >= estimate (>= 1, so never a position past the row),
  // the estimate being the rank-th largest sample. A rank whose estimate lets
  // fewer than `take` keys through, or more than the buffer holds, is
  // replaced by binary search between the ranks known to be too small and
  // too large, and the row filtered again; when no rank is left (a row of
  // many equal keys) the selection runs over the whole row below.
  // Sample rank: about 1.25x (256 threads: a buffer of 2 TOPK entries) or 2x
  // (4096 entries) the expected count of samples above the threshold, plus a
  // margin.
  int rank = THREADS <= 256 ? min(samples, (int)((5 * (int64_t)take * samples) / (4 * (int64_t)cand)) + 8)
                            : min(samples, (int)((2 * (int64_t)take * samples) / cand) + 16);
  int too_few = 0, too_many = samples + 1, n = 0;
  bool buffered = false;
  // A filter pass succeeds only when take <= n <= CAP: with take above the
  // buffer's capacity no pass can, so the row goes straight to the whole-row
  // selection below instead of being streamed by every filter round first.
  for (int round = 0; take <= CAP && round < TK_FILTER_ROUNDS; ++round) {
    const uint32_t estimate = radix_select<THREADS, COMPACT, 2>(
        [&](auto f) {
#pragma unroll
          for (int j = 0; j < SPT; ++j)
            if ((sample_mask >> j) & 1u) f(sample[j]);
        },
        rank, radix, parity, &unused);  // ends with a barrier: every read of `reached` is done
    if (tid == 0) reached = 0;
    __syncthreads();
    // Appends: per step, each lane counts its keys that reach the estimate, a
    // wave scan gives each lane its first slot, and ONE LDS atomic per wave
    // reserves the wave's slots (an atomic with a returned value per key
    // position and wave serialises the pass: prefill 217 -> 192 µs).
    stream_row_steps<THREADS, VEC, FILTER_UNROLL>(
        rsrc, cand, [&](const uint32_t (&keys)[FILTER_UNROLL * 4], int base) {
          int hits = 0;
#pragma unroll
          for (int j = 0; j < FILTER_UNROLL * 4; ++j) hits += keys[j] >= estimate ? 1 : 0;
          const int before = wave_inclusive_scan(hits) - hits;
          const int total = __builtin_amdgcn_readlane(before + hits, 63);
          if (total == 0) return;  // uniform
          int first = 0;
          if (lane == 0) first = atomicAdd(&reached, total);
          int slot = __builtin_amdgcn_readfirstlane(first) + before;
#pragma unroll
          for (int j = 0; j < FILTER_UNROLL * 4; ++j) {
            if (keys[j] >= estimate) {
              if (slot < CAP) {
                buf_key[slot] = keys[j];
                buf_pos[slot] = (Position)stream_position<THREADS, VEC>(base, j);
              }
              ++slot;
            }
          }
        });
    __syncthreads();
    n = reached;
    if (n >= take && n <= CAP) {
      buffered = true;
      break;
    }
    if (n < take)
      too_few = rank;
    else
      too_many = rank;
    rank = too_many > samples ? min(samples, 2 * rank) : (too_few + too_many) / 2;
    if (rank <= too_few || rank >= too_many) break;  // no rank left to try
  }

  // 3. Exact selection, from the buffer when it holds every key that can be
  // taken, else from the row; then the selected keys are marked.
  int need = 0;
  uint32_t threshold = 0;
  if (buffered) {
    threshold = radix_select<THREADS>(
        [&](auto f) {
          for (int i = tid; i < n; i += THREADS) f(buf_key[i]);
        },
        take, radix, parity, &need);
    for (int i = tid; i < n; i += THREADS) {
      const uint32_t k = buf_key[i];
      const int p = buf_pos[i];
      if (k > threshold) atomicOr(&above_bits[p >> 5], 1u << (p & 31));
      else if (k == threshold) atomicOr(&equal_bits[p >> 5], 1u << (p & 31));
    }
  } else {
    threshold = radix_select<THREADS>(
        [&](auto f) {
          stream_row<THREADS, VEC>(rsrc, cand, [&](uint32_t k, int) {
            if (k != 0u) f(k);
          });
        },
        take, radix, parity, &need);
    stream_row<THREADS, VEC>(rsrc, cand, [&](uint32_t k, int p) {
      if (k > threshold) atomicOr(&above_bits[p >> 5], 1u << (p & 31));
      else if (k == threshold) atomicOr(&equal_bits[p >> 5], 1u << (p & 31));
    });
  }
  __syncthreads();

  // 4. Output in position order: thread t owns words [t per, (t + 1) per).
  // Slot of a selected position = keys above the threshold before it +
  // min(equal keys before it, need).
  const int per = (words + THREADS - 1) / THREADS, w0 = min(words, tid * per), w1 = min(words, w0 + per);
  int above_before = 0, equal_before = 0;
  for (int w = w0; w < w1; ++w) {
    above_before += __popc(above_bits[w]);
    equal_before += __popc(equal_bits[w]);
  }
  int totals[2];
  block_exclusive_scan2<THREADS>(above_before, equal_before, scan_scratch, totals);
  for (int w = w0; w < w1; ++w) {
    const uint32_t g = above_bits[w], q = equal_bits[w];
    uint32_t bits = g | q;
    while (bits) {
      const int b = __builtin_ctz(bits);
      bits &= bits - 1;
      const int p = w * 32 + b;
      if ((g >> b) & 1u) {
        const int at = above_before + min(equal_before, need);
        if (at < take) out[at] = p;
        ++above_before;
      } else {
        if (equal_before < need && above_before + equal_before < take) out[above_before + equal_before] = p;
        ++equal_before;
      }
    }
  }
}

// Streaming form, for rows of any length: every digit re-reads the row, and
// the output is written chunk by chunk in position order (one scan per chunk
// of THREADS positions, counting keys equal to the threshold in the high
// half-word and keys above it in the low one).
__global__ __launch_bounds__(TK_STREAM_THREADS) void sparse_topk_stream(TopkArgs a) {
  constexpr int THREADS = TK_STREAM_THREADS;
  __shared__ RadixLds<false> radix;
  __shared__ int scan_scratch[2 * THREADS / 64];
  const int token = blockIdx.x, tid = threadIdx.x;
  const TokenBounds tb = token_bounds(a, token);
  int32_t* out = a.indices + (size_t)token * a.TOPK;
  if (trivial_selection<THREADS>(a, tb, out)) return;
  const float* row = a.scores + (size_t)token * a.C;
  const int cand = tb.cand;
  for (int i = tid; i < TK_BINS; i += THREADS) radix.hist[0][i] = 0u;
  __syncthreads();
  int parity = 0, need = 0;
  const uint32_t threshold = radix_select<THREADS>(
      [&](auto f) {
        for (int i = tid; i < cand; i += THREADS) f(score_key(row[i]));
      },
      tb.take, radix, parity, &need);

  int written = 0, equal_seen = 0;
  for (int base = 0; base < cand; base += THREADS) {
    const int i = base + tid;
    const uint32_t k = i < cand ? score_key(row[i]) : 0u;
    const bool gt = k > threshold, eq = k == threshold;  // k == 0 past the row
    int above = gt ? 1 : 0, equal = eq ? 1 : 0, both[2];
    block_exclusive_scan2<THREADS>(above, equal, scan_scratch, both);
    const int eq_left = max(0, need - equal_seen);  // equal keys still to take
    const int at = written + above + min(equal, eq_left);
    if ((gt || (eq && equal < eq_left)) && at < tb.take) out[at] = i;
    written += both[0] + min(both[1], eq_left);
    equal_seen += both[1];
    if (written >= tb.take) break;  // uniform: every thread sees the same totals
  }
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
  const bool vec = (params->C % 4 == 0) && (reinterpret_cast<uintptr_t>(scores) % 16 == 0);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)a.T);
  a.words = (int32_t)((a.C + 31) / 32);
  // Buffer: rows up to 32K positions (16-bit positions) hold 2 TOPK entries,
  // between 1024 and 8192, so that little of a CU's LDS is spent on it at the
  // usual TOPK; longer rows hold TK_WIDE_CAP.
  a.cap = a.C <= 32768 ? (int32_t)std::min<int64_t>(8192, std::max<int64_t>(1024, ((int64_t)a.TOPK * 2 + 255) / 256 * 256))
                       : TK_WIDE_CAP;
  if (a.C <= TK_FILTER_MAX_C) {
    const size_t dynamic_bytes = 2 * 4 * (size_t)a.words + (a.C <= 32768 ? (size_t)a.cap * 6 : 0);
    // Rows up to 32K positions: 256 threads, more workgroups per CU; longer
    // rows: 1024 threads, more loads in flight per row.
    if (a.C <= 32768) {
      if (vec)
        hipLaunchKernelGGL((sparse_topk_filter<256, true>), grid, dim3(256), dynamic_bytes, s, a);
      else
        hipLaunchKernelGGL((sparse_topk_filter<256, false>), grid, dim3(256), dynamic_bytes, s, a);
    } else {
      if (vec)
        hipLaunchKernelGGL((sparse_topk_filter<1024, true>), grid, dim3(1024), dynamic_bytes, s, a);
      else
        hipLaunchKernelGGL((sparse_topk_filter<1024, false>), grid, dim3(1024), dynamic_bytes, s, a);
    }
  } else {
    hipLaunchKernelGGL(sparse_topk_stream, grid, dim3(TK_STREAM_THREADS), 0, s, a);
  }
  return (int)hipGetLastError();
}
