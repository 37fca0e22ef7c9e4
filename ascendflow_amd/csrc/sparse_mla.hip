// Sparse MLA forward for gfx950: top-k compressed-KV plus sliding-window
// gather, QK^T, online softmax with one sink per head, PV, in ONE kernel.
//
// Reference operator: examples/sparse_attention/attention.py:210-525 (sparse_mla)
// with the gather helpers of examples/sparse_attention/gather.py:8-131. The
// reference splits the work over a Cube core and two Vector cores that hand
// Score/P/PV and the gathered rows to each other through double/triple-slot
// GM workspaces. Here one workgroup owns one (token, BM-head tile):
//
//   1. resolve the token's request and window/compressed bounds
//      (gather.py:8-35, attention.py:339-341) and compact every selected row
//      (window positions, then compressed ranks, duplicates kept) into an LDS
//      row list of physical row ids. With a workspace and at least two work
//      items per CU, a plan kernel does this for every token first and a
//      persistent form (sparse_mla_persistent_kernel) streams the tokens of
//      each CU through one pipeline, so the dependent global round trips
//      and the pipeline fill no longer idle the matrix cores at token starts;
//   2. stream the listed rows through a 3- or 4-stage ring of XOR-swizzled
//      LDS tiles of CHUNK rows with the load-to-LDS path
//      (global_load_lds_dwordx4, one wave load per 1 KiB row when D = 512);
//   3. score waves (16 heads each, all D features of Q resident in registers):
//      S^T[rows, heads] = KV * Q^T on v_mfma_f32_16x16x32_{bf16,f16}, FP32
//      online softmax in the exp2 domain (the sink seeds the running max and
//      contributes e^(sink-m) once), P rounded to the storage dtype
//      (round-to-nearest-even) and handed over through LDS;
//   4. output waves (all heads, D/NP features each): O^T[d, heads] +=
//      V^T * P^T, V^T fragments from the same LDS rows through
//      ds_read_b64_tr_b16;
//   5. O = O_acc * (1 / l), rounded to the storage dtype. Keys of a short
//      last round may instead be split over several workgroups by list
//      chunks; each part stores its normalised output with its running max
//      and denominator, and sparse_merge_kernel combines the parts.
//
// K and V are the same gathered rows; each row is read from global memory
// once per workgroup and from LDS once per score wave and once per output wave.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <utility>

#include "common.h"
#include "../../include/ascendflow_amd.h"

namespace afa {

constexpr int CHUNK = 32;                 // rows per LDS stage
constexpr int MAX_PARTS = 8;              // most parts a token's chunk list is split into
constexpr uint32_t CMP_BIT = 0x80000000u; // row-list tag: row lives in cmp_kv
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// Natural-log normaliser of a head's softmax: ln(sum_j e^(s_j) + e^sink), from
// the running max m (log2 units, scores pre-scaled by log2 e) and the
// denominator l relative to it.
__device__ __forceinline__ float lse_of(float m, float l) { return (m + __log2f(l)) * LN2; }

struct SparseArgs {
  const void* q;
  const void* ori_kv;
  const void* cmp_kv;
  const int32_t* indices;
  const int32_t* ori_table;
  const int32_t* cmp_table;
  const int32_t* cu;
  const int32_t* seq_ori;
  const int32_t* seq_cmp;
  const int32_t* residual;
  const int32_t* ori_topk_length;
  const float* sinks;
  void* out;
  float* lse;            // optional [T][H] natural-log softmax normaliser, or null
  int32_t* debug_rows;
  uint32_t* plan_rows;   // workspace: [T][list_pad] padded row lists, or null
  int32_t* plan_count;   // workspace: [T] selected rows per token
  void* partials;        // workspace: [split keys][parts][output waves] records (store_record)
  int32_t B, T, H, D, PAGE, RATIO, table_width, ori_blocks, cmp_blocks, WINDOW, TOPK, S, BM;
  int32_t list_pad;      // row-list capacity: WINDOW + TOPK rounded up to 256 (whole KiB)
  int32_t parts;         // parts each split (token, head tile) key is divided into (one-item kernel)
  int32_t split_from;    // first split (token, head tile) key; keys below it run whole
  int32_t ring;          // KV ring tiles of the persistent kernel (3 or 4)
  int32_t stream_kv;     // few query tokens per request: non-temporal KV, Q and O accesses (D = 512)
  float scale;
};

struct Geometry {
  int batch, right, visible, cutoff, count_cmp;
};

// Request of a token: upper_bound(cu_seqlens_q[0..B], token) - 1, i.e. the
// last b in [0, B) with cu[b] <= token (gather.py:10-21; empty requests have
// cu[b] == cu[b+1] and are skipped). Binary search, one thread.
__device__ __forceinline__ int request_by_search(const SparseArgs& a, int token) {
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
  return lo;
}

// query_metadata (gather.py:8-35) and the compressed bound (attention.py:339-341)
// of a token whose request is `batch`.
// The request's inputs of the geometry: cu[b], cu[b + 1], seq_ori[b],
// seq_cmp[b], residual[b].
struct RequestInputs {
  int begin, next, seq_ori, seq_cmp, residual;
};
__device__ __forceinline__ RequestInputs request_inputs(const SparseArgs& a, int b) {
  return RequestInputs{a.cu[b], a.cu[b + 1], a.seq_ori[b], a.seq_cmp[b], a.residual[b]};
}
// narrowed = ori_topk_length[token].
__device__ __forceinline__ Geometry geometry_of(const SparseArgs& a, int token, int batch, const RequestInputs& r,
                                                int narrowed) {
  Geometry g;
  g.batch = batch;
  const int begin = r.begin, count = r.next - begin, offset = token - begin;
  g.right = max(0, r.seq_ori - count + offset + 1);
  int visible = min(a.WINDOW, g.right);
  if (narrowed > 0) visible = min(visible, narrowed);
  g.visible = visible;
  const int available = r.seq_cmp;
  const int end = available * a.RATIO + r.residual;
  g.cutoff = max(0, end - count + offset + 1) / a.RATIO;
  g.count_cmp = max(0, min(a.TOPK, min(available, g.cutoff)));
  return g;
}
__device__ __forceinline__ Geometry token_geometry(const SparseArgs& a, int token, int batch) {
  return geometry_of(a, token, batch, request_inputs(a, batch), a.ori_topk_length[token]);
}

// Resolve gather slot s of a token (window slot s < WINDOW, else compressed
// rank s - WINDOW) to a tagged physical row. Returns false for an unused slot
// (gather.py:116-127; window rows: gather.py:38-60). Page-table entries that
// point outside the cache are treated as unused rather than read.
__device__ __forceinline__ bool resolve_slot(const SparseArgs& a, const Geometry& g, int token,
                                             int s, uint32_t& entry) {
  const int* table_row;
  if (s < a.WINDOW) {
    if (s >= g.visible) return false;
    const int position = g.right - g.visible + s;
    table_row = a.ori_table + (size_t)g.batch * a.table_width;
    const int column = min(position / a.PAGE, a.table_width - 1);
    const int block = table_row[column];
    if (block < 0 || block >= a.ori_blocks) return false;
    entry = (uint32_t)(block * a.PAGE + position % a.PAGE);
    return true;
  }
  const int rank = s - a.WINDOW;
  if (rank >= g.count_cmp) return false;
  const int index = a.indices[(size_t)token * a.TOPK + rank];
  if (index < 0 || index >= g.cutoff) return false;
  const int cpage = a.PAGE / a.RATIO;
  table_row = a.cmp_table + (size_t)g.batch * a.table_width;
  const int column = min(index / cpage, a.table_width - 1);
  const int block = table_row[column];
  if (block < 0 || block >= a.cmp_blocks) return false;
  entry = CMP_BIT | (uint32_t)(block * cpage + index % cpage);
  return true;
}

template <typename T>
__device__ __forceinline__ const T* row_pointer(const SparseArgs& a, uint32_t entry) {
  const T* base = (const T*)((entry & CMP_BIT) ? a.cmp_kv : a.ori_kv);
  return base + (size_t)(entry & ~CMP_BIT) * a.D;
}

// Resolves the selected rows of `token` into row_list (LDS) in slot order
// (window positions, then compressed ranks) and returns their count. Every
// one of the NTH threads of the workgroup must call it (workgroup barriers);
// wave_count is LDS scratch of [GP][NTH / 64], request_scratch of
// [NTH / 64 + 5]. With B <= NTH, two dependent global round trips: the
// request count, the compressed indices and every request's geometry inputs
// (thread b those of request b; the thread of the token's request hands them
// to the others through LDS), then the compressed and the window page lookups
// together (gather.py:8-60, 116-127; attention.py:339-341). Larger B loads
// the geometry inputs once the request is known, and the window lookups wait
// for them (three round trips). GP passes of NTH slots go together, so
// WINDOW + TOPK <= GP * NTH takes one such sequence.
template <int NTH, int GP>
__device__ __forceinline__ int resolve_rows(const SparseArgs& a, int token, uint32_t* row_list,
                                            int (*wave_count)[NTH / 64], int* request_scratch,
                                            Geometry& geo) {
  constexpr int NWV = NTH / 64;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  // Request of the token: cu is non-decreasing with cu[0] = 0 <= token, so it
  // is #{b in [0, B): cu[b] <= token} - 1 (gather.py:10-21; empty requests
  // have cu[b] == cu[b+1] and are skipped).
  int below = 0;
  for (int b = tid; b < a.B; b += NTH) below += a.cu[b] <= token ? 1 : 0;
  const bool early = a.B <= NTH;  // uniform
  RequestInputs mine{0, 0, 0, 0, 0};
  if (early && tid < a.B) mine = request_inputs(a, tid);
  const int narrowed = a.ori_topk_length[token];
  int index[GP];
  auto load_indices = [&](int s0) {
#pragma unroll
    for (int k = 0; k < GP; ++k) {
      const int rank = s0 + k * NTH + tid - a.WINDOW;
      index[k] = (rank >= 0 && rank < a.TOPK) ? a.indices[(size_t)token * a.TOPK + rank] : -1;
    }
  };
  load_indices(0);
  below = __builtin_amdgcn_readlane(wave_inclusive_scan(below), 63);  // the wave's sum
  if (lane == 0) request_scratch[wave] = below;
  __syncthreads();
  int requests = 0;
#pragma unroll
  for (int w = 0; w < NWV; ++w) requests += request_scratch[w];
  // At least request 0: cu_seqlens_q starts at 0 <= token, and an input that
  // breaks that still reads request 0's tables, never memory before them.
  const int batch = max(requests - 1, 0);

  // The compressed page lookups need only the request and the indices, so
  // they go out first; the window lookups need the geometry.
  const int cpage = a.PAGE / a.RATIO;
  const int* cmp_row = a.cmp_table + (size_t)batch * a.table_width;
  const int* ori_row = a.ori_table + (size_t)batch * a.table_width;
  int cblock[GP];
  auto load_cmp_blocks = [&]() {
#pragma unroll
    for (int k = 0; k < GP; ++k)
      cblock[k] = index[k] >= 0 ? cmp_row[min(index[k] / cpage, a.table_width - 1)] : -1;
  };
  load_cmp_blocks();
  if (early) {
    int* inputs = request_scratch + NWV;
    if (tid == batch) {
      inputs[0] = mine.begin;
      inputs[1] = mine.next;
      inputs[2] = mine.seq_ori;
      inputs[3] = mine.seq_cmp;
      inputs[4] = mine.residual;
    }
    __syncthreads();
    geo = geometry_of(a, token, batch, RequestInputs{inputs[0], inputs[1], inputs[2], inputs[3], inputs[4]},
                      narrowed);
  } else {
    geo = geometry_of(a, token, batch, request_inputs(a, batch), narrowed);
  }
  const int slots = a.WINDOW + geo.count_cmp;
  // Slot s (window slot s < WINDOW, else compressed rank s - WINDOW) resolves
  // to a tagged physical row as in resolve_slot (gather.py:38-60, 116-127).
  int n_rows = 0;
  for (int s0 = 0; s0 < slots; s0 += GP * NTH) {
    if (s0 > 0) {
      load_indices(s0);
      load_cmp_blocks();
    }
    uint32_t entry[GP];
    bool valid[GP];
#pragma unroll
    for (int k = 0; k < GP; ++k) {
      const int s = s0 + k * NTH + tid;
      valid[k] = false;
      entry[k] = 0;
      if (s < a.WINDOW) {
        if (s < geo.visible) {
          const int position = geo.right - geo.visible + s;
          const int block = ori_row[min(position / a.PAGE, a.table_width - 1)];
          valid[k] = block >= 0 && block < a.ori_blocks;
          entry[k] = (uint32_t)(block * a.PAGE + position % a.PAGE);
        }
      } else if (s < slots) {
        valid[k] = index[k] >= 0 && index[k] < geo.cutoff && cblock[k] >= 0 && cblock[k] < a.cmp_blocks;
        entry[k] = CMP_BIT | (uint32_t)(cblock[k] * cpage + index[k] % cpage);
      }
    }
    // Order-preserving compaction of the GP passes, one pair of barriers.
    uint64_t mask[GP];
#pragma unroll
    for (int k = 0; k < GP; ++k) {
      mask[k] = __ballot(valid[k]);
      if (lane == 0) wave_count[k][wave] = __popcll(mask[k]);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < GP; ++k) {
      int before = 0, total = 0;
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const int c = wave_count[k][w];
        before += w < wave ? c : 0;
        total += c;
      }
      if (valid[k]) row_list[n_rows + before + __popcll(mask[k] & ((1ull << lane) - 1ull))] = entry[k];
      n_rows += total;
    }
    __syncthreads();
  }
  return n_rows;
}

// A token's chunk list split into P parts: part p covers list chunks
// [p * n / P, (p + 1) * n / P) of the token's n = max(1, ceil(count / CHUNK))
// chunks. An empty part (n < P) streams one fully masked chunk (list chunk 0),
// so every work item has at least one chunk and one partial result.
struct PartRange {
  int first;  // first list chunk of the part
  int n;      // list chunks of the part; 0 for the masked placeholder
};
__device__ __forceinline__ PartRange part_range(int count, int part, int parts) {
  const int nch = max(1, (count + CHUNK - 1) / CHUNK);
  const int c0 = part * nch / parts, c1 = (part + 1) * nch / parts;
  return PartRange{c0, c1 - c0};
}

// Plan kernel: one workgroup per token writes the token's row list, padded
// with its first row to a whole number of CHUNK-row chunks, and the count.
template <int NTH>
__global__ __launch_bounds__(NTH) void sparse_plan_kernel(SparseArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint32_t plan_list[];
  // One wave per token, ten passes of 64 slots: WINDOW + TOPK = 640 in one
  // round-trip sequence. The kernel is latency-bound (two or three dependent
  // round trips per token); one-wave workgroups let every token of a Q8K
  // prefill be resident at once (four waves per token took ~4 rounds of
  // residency: prefill 0.7-1.2% slower).
  constexpr int GP = 10;
  __shared__ int wave_count[GP][NTH / 64];
  __shared__ int request_scratch[NTH / 64 + 5];
  const int token = blockIdx.x;
  Geometry geo;
  const int n = resolve_rows<NTH, GP>(a, token, plan_list, wave_count, request_scratch, geo);
  // An empty list becomes one chunk of row 0 of ori_kv (every score masked),
  // so every token has at least one chunk to stream.
  const int padded = n > 0 ? (n + CHUNK - 1) / CHUNK * CHUNK : CHUNK;
  uint32_t* dst = a.plan_rows + (size_t)token * a.list_pad;
  for (int r = threadIdx.x; r < padded; r += NTH) dst[r] = n > 0 ? plan_list[r < n ? r : 0] : 0u;
  if (threadIdx.x == 0) a.plan_count[token] = n;
}

// Partial result of one part of a split key, for sparse_merge_kernel: output
// wave ow's record holds its O slice normalised by the part's own denominator
// and rounded to the storage dtype, as x4 at (ht * PVT + t) * 64 + lane (head
// 16 ht + (lane & 15), features ow * DPV + 16 t + 4 (lane >> 4) + 0..3), then
// the part's running max (log2 units) and denominator of the BMH heads.
template <int DT> __host__ __device__ constexpr size_t record_bytes(int bmh, int dpv) {
  return (size_t)bmh * dpv * sizeof(typename B16<DT>::scalar) + 2 * (size_t)bmh * sizeof(float);
}
template <int DT, int NQ, int NP, int DPV>
__device__ __forceinline__ void store_record(const SparseArgs& a, int split_key, int part, int ow,
                                             const f32x4 (&o)[NQ][DPV / 16], const float* linv,
                                             const float (*ml)[16 * NQ], int lane) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x4 x4;
  constexpr int BMH = 16 * NQ, PVT = DPV / 16;
  char* rec = (char*)a.partials + (((size_t)split_key * a.parts + part) * NP + ow) * record_bytes<DT>(BMH, DPV);
#pragma unroll
  for (int ht = 0; ht < NQ; ++ht) {
    const float inv = linv[16 * ht + (lane & 15)];
#pragma unroll
    for (int t = 0; t < PVT; ++t) {
      x4 v;
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = (scalar)(o[ht][t][k] * inv);
      *(x4*)(rec + (size_t)((ht * PVT + t) * 64 + lane) * sizeof(x4)) = v;
    }
  }
  float* stats = (float*)(rec + (size_t)BMH * DPV * sizeof(scalar));
  if (lane < BMH) {
    stats[lane] = ml[0][lane];
    stats[BMH + lane] = ml[1][lane];
  }
}

// Lazy rescaling threshold (log2 units): the running max used for exp2 is only
// raised, and O/l rescaled, once some head's max exceeds it by more than
// TAU, so P stays <= 2^TAU; the final O/l is independent of the reference point.
constexpr float TAU = 8.0f;

// Stores one 16-head tile of O, held as the PV accumulators hold it (lane
// (i16, g) has features 16t + 4g + 0..3 of head i16, t < DPV / 16), scaled by
// inv and rounded, through a wave-private LDS stage, so that each global store
// writes whole DPV * 2-byte head-row slices (full cache lines). Stored straight
// from the accumulators, every instruction would write 16 scattered 32-byte
// pieces; measured on prefill Q8K, that pattern costs ~9% of the kernel.
// Head row h of the stage starts at stage + h * STAGE_ROW and holds 16-byte
// unit u of the head row at unit (unit_base + u) ^ (h & SWZ): packed
// (STAGE_ROW = DPV * 2, unit_base 0, SWZ = units - 1), or the wave's own
// feature units of a KV ring tile (STAGE_ROW = the tile's row bytes, unit_base
// = the wave's first feature unit, SWZ = 15: the tile's own swizzle). The
// stage is only touched by this wave, whose LDS operations complete in order.
// NT: non-temporal global stores (the write-once O leaves the L2 to the KV
// rows that other work items of the request read; decode 63.4 -> 61.8 µs,
// while the persistent prefill kernel measured ~1% slower with them).
template <int DT, int DPV, int STAGE_ROW = DPV * 2, int SWZ = DPV / 8 - 1, bool NT = false>
__device__ __forceinline__ void store_head_tile(uint32_t stage, uint32_t unit_base, const f32x4 (&o)[DPV / 16],
                                                float inv, typename B16<DT>::scalar* out, size_t head_stride,
                                                int lane) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x4 x4;
  constexpr int PVT = DPV / 16;
  constexpr int UR = DPV / 8;            // 16-byte units per head row
  constexpr int HPI = 1024 / (DPV * 2);  // head rows per 1 KiB wave access
  static_assert((UR & (UR - 1)) == 0 && 16 % HPI == 0, "power-of-two head rows of at most 1 KiB");
  static_assert(STAGE_ROW >= DPV * 2 && (SWZ == UR - 1 || SWZ == 15), "stage rows hold a head row each");
  const int i16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < PVT; ++t) {
    x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = (scalar)(o[t][k] * inv);
    const uint32_t unit = (unit_base + (uint32_t)(2 * t + (g >> 1))) ^ (uint32_t)(i16 & SWZ);
    *(AFA_LDS x4*)(uintptr_t)(stage + (uint32_t)(i16 * STAGE_ROW) + unit * 16u + (uint32_t)(g & 1) * 8u) = v;
  }
#pragma unroll
  for (int r = 0; r < 16 / HPI; ++r) {
    const int h = r * HPI + lane / UR, u = lane % UR;
    const uint32_t unit = (unit_base + (uint32_t)u) ^ (uint32_t)(h & SWZ);
    const u32x4 w = *(const AFA_LDS u32x4*)(uintptr_t)(stage + (uint32_t)(h * STAGE_ROW) + (unit << 4));
    u32x4* dst = (u32x4*)((char*)(out + (size_t)h * head_stride) + u * 16);
    if constexpr (NT)
      __builtin_nontemporal_store(w, dst);
    else
      *dst = w;
  }
}

constexpr int LOOK = 4;     // V^T fragment lookahead (16-feature tiles) of an output wave
constexpr int LOOK_QK = 5;  // KV fragment lookahead (k-steps) of a score wave

// Workgroup = one (token, BM-head tile), BM = 16 * NQ, split by role:
//  - score wave q < NQ owns heads [16q, 16q + 16) with all D features of Q
//    resident: S^T = KV * Q^T for the chunk, FP32 online softmax, and the
//    rounded P written to LDS in the MFMA B-operand layout;
//  - output wave p owns features [p * D/NP, +D/NP) of all BM heads:
//    O^T += V^T * P^T, so every V^T fragment read from LDS feeds NQ MFMAs.
// No partial scores are exchanged, each KV row is read from LDS once per score
// wave and once per output wave, and the softmax VALU work sits on score waves
// only. Waves w and w + 4 of a 512-thread workgroup share a SIMD (measured
// dispatch order), so with NQ = NP = 4 every SIMD runs one wave of each role
// and their LDS, VALU and MFMA phases interleave.
//
// Software pipeline, one barrier per step i = 0..chunks:
//   wait KV(i) -> barrier -> fetch KV(i + NS - 2) -> score waves: QK(i),
//   softmax(i), P(i) -> LDS slot i&1; output waves: PV(i-1) from slot (i-1)&1.
// KV uses a ring of NS tiles (3: one chunk in flight; 4: two, for streams whose
// rows come from HBM): during step i the score waves read tile i and the output
// waves tile i-1, so the fetch at the top of step i never overwrites a tile
// still in use. With D = 512 and NQ = NP = 4 the output waves issue the whole
// fetch (8 rows each) and the score waves, whose step is the longer one, only
// wait at the barrier (decode B64 x 6 ~2% faster than every wave fetching 4
// rows); other shapes spread the fetch over every wave.
// STREAM_KV: KV row loads are non-temporal as well (Q and O always are), for
// calls whose requests have few query tokens.
template <int DT, int D, int NQ, int NP, int NS, bool STREAM_KV = false>
__global__ __launch_bounds__((NQ + NP) * 64) void sparse_mla_kernel(SparseArgs a) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x8 x8;
  typedef typename B16<DT>::x4 x4;
  constexpr int NW = NQ + NP;
  constexpr int NT = NW * 64;
  constexpr int BMH = 16 * NQ;                 // heads per workgroup
  constexpr int UNITS = D / 8;                 // 16-byte units per row
  constexpr int PIECES = CHUNK * UNITS / NT;   // 16-byte loads per thread per chunk
  constexpr int ROW_BYTES = D * 2;
  constexpr int QK_STEPS = D / 32;             // k-steps of a score wave
  constexpr int DPV = D / NP;                  // features per output wave
  constexpr int PVT = DPV / 16;                // 16-feature tiles per output wave
  static_assert(CHUNK * UNITS % NT == 0, "chunk must split evenly over the block");
  static_assert(UNITS >= 16, "swizzle needs at least 16 units per row");
  static_assert(DPV % 16 == 0 && (PVT <= 8 || (DPV / 8) % 16 == 0), "output feature range");

  constexpr int AHEAD = NS - 2;  // chunks fetched ahead of the score waves
  static_assert(NS == 3 || NS == 4, "KV ring of 3 or 4 tiles");
  __shared__ __attribute__((aligned(16))) uint8_t kv_lds[NS][CHUNK * ROW_BYTES];
  __shared__ __attribute__((aligned(16))) u32x4 p_lds[2][NQ][64];  // P in B-operand layout
  __shared__ float alpha_lds[2][BMH];   // O rescale factor per head, valid when flagged
  __shared__ __attribute__((aligned(16))) int flag_lds[2][4];  // score wave q raised its running max
  __shared__ float linv_lds[BMH];       // 1 / softmax denominator per head
  __shared__ float ml_lds[2][BMH];      // running max (log2 units) and denominator per head
  __shared__ int wave_count[2][NW];
  extern __shared__ __attribute__((aligned(16))) uint32_t row_list[];  // round_up(WINDOW + TOPK, CHUNK) entries

  const int tid = threadIdx.x;
  // The wave index is uniform; readfirstlane lets the compiler see that, so
  // branches on the wave's role are scalar branches.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 4, i16 = lane & 15;
  const bool scorer = wave < NQ;
  const int head_tiles = a.H / a.BM;
  // Whole keys and split parts are each spread XCD-contiguously on their own
  // (when split_from is a multiple of the 8 XCDs, the hardware block ids of the
  // two segments then fall on the same XCD pattern): over the whole grid, the
  // XCDs holding the low logical ids would get every whole key and the others
  // only parts.
  const uint32_t s0 = (uint32_t)a.split_from;  // <= gridDim.x
  const int logical = (int)((s0 & 7u) != 0 ? xcd_contiguous(blockIdx.x, gridDim.x)
                            : blockIdx.x < s0 ? xcd_contiguous(blockIdx.x, s0)
                                              : s0 + xcd_contiguous(blockIdx.x - s0, gridDim.x - s0));
  // Work item: key (token, head tile) `logical` below split_from, whole; from
  // split_from on, item split_from + k * parts + p is part p of key
  // split_from + k (a contiguous range of its list chunks, merged afterwards).
  const int S0 = a.split_from, P = a.parts;
  const bool split = logical >= S0;
  const int key = split ? S0 + (logical - S0) / P : logical;
  const int part = split ? (logical - S0) % P : 0;
  const int token = key / head_tiles;
  const int head0 = (key % head_tiles) * a.BM;

  // ---- 1-2. the token's row list in LDS and Q. Q (BMH contiguous rows of D features) is copied with the
  // load-to-LDS path in coalesced 1 KiB wave loads into ring tiles 1 and 2,
  // which stay unused until the first pipeline step, with the KV rows' unit
  // swizzle; each score wave then reads its B-operand fragments (S^T = KV *
  // Q^T) from there once. Loading the fragments straight into registers
  // touches 64-byte pieces of 16 rows per wave load and stalls the issue of
  // every other load of the workgroup for thousands of cycles. Q is read once:
  // the loads are non-temporal, like the O stores.
  const uint32_t q_lds = lds_address(kv_lds[NS - 2]);
  constexpr int Q_LOADS = BMH * ROW_BYTES / 1024;  // 1 KiB wave loads of the Q tile
  static_assert(BMH * ROW_BYTES <= 2 * CHUNK * ROW_BYTES, "Q tile must fit ring tiles 1 and 2");
  auto copy_q = [&]() {
    const char* q_src = (const char*)a.q + ((size_t)token * a.H + head0) * ROW_BYTES;
#pragma unroll
    for (int k0 = 0; k0 < Q_LOADS; k0 += NW) {
      const int k = k0 + wave;
      if (Q_LOADS % NW == 0 || k < Q_LOADS) {
        const int pos = k * 64 + lane;  // 16-byte unit position in the tile
        const int r = pos / UNITS, u = pos % UNITS;
        const uint32_t off = (uint32_t)(r * ROW_BYTES + ((u ^ (r & 15)) << 4));
        __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                         :: "s"(q_lds + (uint32_t)k * 1024u), "v"(off), "s"(q_src) : "memory");
      }
    }
  };
  __shared__ int request_scratch[NW + 5];
  int n_rows;
  {
    // Q does not depend on the row list: its copy goes out first and lands
    // while the rows are resolved (two or three dependent round trips).
    copy_q();
    Geometry geo;
    n_rows = resolve_rows<NT, 2>(a, token, row_list, wave_count, request_scratch, geo);
    // Pad the last chunk with a real row so every load is unconditional; the
    // padded rows get -inf scores (P = 0) below.
    const int padded = (n_rows + CHUNK - 1) / CHUNK * CHUNK;
    if (tid < padded - n_rows) row_list[n_rows + tid] = row_list[0];
    // A part of an empty selection streams one masked chunk of ori row 0.
    if (split && n_rows == 0 && tid < CHUNK) row_list[tid] = 0u;
    if (a.debug_rows != nullptr && head0 == 0 && part == 0) {
      // The compacted list this workgroup streams, entry r < n_rows as
      // (cache, physical row), then (-1, -1). Entries below n_rows are final
      // (resolve_rows ended with a barrier); the padding writes above touch
      // only entries from n_rows on.
      for (int r = tid; r < a.S; r += NT) {
        int2 v = make_int2(-1, -1);
        if (r < n_rows) {
          const uint32_t e = row_list[r];
          v = make_int2((e & CMP_BIT) ? 1 : 0, (int)(e & ~CMP_BIT));
        }
        ((int2*)a.debug_rows)[(size_t)token * a.S + r] = v;
      }
    }
    block_barrier();
  }
  // This item's list chunks: all of them, or its part's range (an empty part
  // streams one fully masked chunk of list chunk 0).
  const PartRange range = split ? part_range(n_rows, part, P) : PartRange{0, (n_rows + CHUNK - 1) / CHUNK};
  const bool placeholder = split && range.n == 0;
  const int chunks = placeholder ? 1 : range.n;
  auto list_chunk = [&](int i) { return placeholder ? 0 : range.first + i; };

  // ---- 3. KV movement: global -> LDS through the load-to-LDS path ------------
  // global_load_lds_dwordx4 writes one wave's 64 x 16 bytes contiguously at the
  // LDS address in M0. The XOR swizzle is applied on the global side (the lane
  // that lands on unit position u of row r loads unit u ^ (r & 15)), so LDS
  // holds the swizzled rows without VGPR staging or ds_write traffic. M0 is
  // set inside the same asm statement; nothing else in this kernel uses M0.
  // Completion is tracked with vmcnt: when a step waits, the only vector
  // memory loads in flight are the previous fetch's.
  // With D = 512 one wave load covers exactly one 1 KiB row, so a fetching
  // wave takes FPW consecutive rows whose list entries and addresses are
  // wave-uniform (scalar registers), and the entries are read one step ahead.
  // OWN_FETCH: only the output waves fetch (FPW = CHUNK / NP rows each).
  constexpr bool ROW_LOADS = (UNITS == 64);
  constexpr bool OWN_FETCH = ROW_LOADS && NQ == 4 && NP == 4;
  constexpr int FPW = OWN_FETCH ? CHUNK / NP : PIECES;
  const bool fetcher = !OWN_FETCH || !scorer;
  const int fw = OWN_FETCH ? wave - NQ : wave;  // this wave's index among the fetching waves
  const char* ori = (const char*)a.ori_kv;
  const char* cmp = (const char*)a.cmp_kv;
  const uint32_t kv_base = lds_address(kv_lds[0]);
  auto tile_address = [&](int chunk) {
    return opaque_uniform(kv_base + (uint32_t)(chunk % NS) * (CHUNK * ROW_BYTES));
  };
  uint32_t unit_offset[FPW];  // ROW_LOADS: byte offset of the unit this lane loads
#pragma unroll
  for (int p = 0; p < FPW; ++p) unit_offset[p] = (uint32_t)((lane ^ ((fw * FPW + p) & 15)) << 4);
  uint32_t entry_next[FPW];
  auto read_entries = [&](int chunk) {
#pragma unroll
    for (int p = 0; p < FPW; ++p) entry_next[p] = row_list[list_chunk(chunk) * CHUNK + fw * FPW + p];
  };
  auto fetch = [&](int chunk) {
    const uint32_t tile = tile_address(chunk);
    if constexpr (ROW_LOADS) {
#pragma unroll
      for (int p = 0; p < FPW; ++p) {
        const int r = fw * FPW + p;
        const uint32_t e = __builtin_amdgcn_readfirstlane(entry_next[p]);
        const char* row = ((e & CMP_BIT) ? cmp : ori) + (size_t)(e & ~CMP_BIT) * ROW_BYTES;
        const uint32_t dst = tile + (uint32_t)(r * ROW_BYTES);
        if constexpr (STREAM_KV)
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                           :: "s"(dst), "v"(unit_offset[p]), "s"(row) : "memory");
        else
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                           :: "s"(dst), "v"(unit_offset[p]), "s"(row) : "memory");
      }
      if (chunk + 1 < chunks) read_entries(chunk + 1);
    } else {
#pragma unroll
      for (int p = 0; p < PIECES; ++p) {
        const int flat = tid + p * NT;
        const int r = flat / UNITS, upos = flat % UNITS;
        const uint32_t e = row_list[list_chunk(chunk) * CHUNK + r];
        const char* src = ((e & CMP_BIT) ? cmp : ori) + (size_t)(e & ~CMP_BIT) * ROW_BYTES + ((upos ^ (r & 15)) << 4);
        const uint32_t dst = tile + (uint32_t)((wave * 64 + p * NT) * 16);
        if constexpr (STREAM_KV)
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt"
                           :: "s"(dst), "v"(src) : "memory");
        else
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                           :: "s"(dst), "v"(src) : "memory");
      }
    }
  };
  // Pipeline step i: wait for KV(i), barrier, fetch KV(i + AHEAD), then the
  // role's work. Loads complete in issue order, so KV(i) has landed once at
  // most the younger batch (KV(i + 1), with a 4-tile ring) is in flight.
  if (fetcher && chunks > 0) {
    if constexpr (ROW_LOADS) read_entries(0);
    fetch(0);
    if (AHEAD > 1 && chunks > 1) {
      fetch(1);
      // Q has landed once at most the loads of the two prologue fetches are in flight.
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * FPW) & 15) | (((2 * FPW) >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70 | (FPW & 15) | ((FPW >> 4) << 14));
    }
  } else {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's Q loads
  }
  block_barrier();
  // Score wave fragments: this lane holds head 16 * wave + i16 (tile row r),
  // features 32j + 8g .. +7, i.e. unit 4j + g of row r, stored at unit
  // (4j + g) ^ (r & 15). Its ring tiles are overwritten only after the next barrier.
  const int qhead = head0 + 16 * wave + i16;   // score wave: this lane's head
  x8 qf[QK_STEPS];
  if (scorer) {
    const int r = 16 * wave + i16;
#pragma unroll
    for (int j = 0; j < QK_STEPS; ++j)
      qf[j] = *lds_at<x8>(q_lds + (uint32_t)(r * ROW_BYTES + (((4 * j + g) ^ (r & 15)) << 4)));
  }
  auto step_begin = [&](int i) {
    if (fetcher && i < chunks) {
      if (AHEAD > 1 && i + 1 < chunks)
        __builtin_amdgcn_s_waitcnt(0x0F70 | (FPW & 15) | ((FPW >> 4) << 14));
      else
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    block_barrier();
    if (fetcher && i + AHEAD < chunks) fetch(i + AHEAD);
  };

  // The swizzle only permutes units within aligned groups of 16 (256 bytes),
  // so a fragment address is a per-lane base plus a compile-time offset.
  if (scorer) {
    // ---- 4a. score wave: QK, online softmax, P -------------------------------
    // Here the score waves' step (QK and softmax, plus their share of the
    // fetch unless OWN_FETCH) is the longer one: they get the higher wave
    // priority (the output waves' instead made decode 6% slower).
    __builtin_amdgcn_s_setprio(2);
    // The running max (log2 units) starts at the sink and is raised (with l
    // rescaled here and O rescaled by the output waves) only when a head's max
    // exceeds it by more than TAU. This lane holds S^T rows sigma(4g+i) and
    // 16 + sigma(4g+i) of head qhead.
    float m_run = a.sinks[qhead] * LOG2E;
    float l_run = (g == 0 && part == 0) ? 1.0f : 0.0f;  // e^(sink - m), once per head and token
    const float scale_log2 = a.scale * LOG2E;
    const int ra = sigma(i16);           // KV fragment row inside a 16-row tile
    uint32_t qk_base[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) qk_base[b] = (uint32_t)(ra * ROW_BYTES + (((4 * b + g) ^ (ra & 15)) << 4));

    for (int i = 0; i <= chunks; ++i) {
      step_begin(i);
      if (i == chunks) break;
      // S^T of chunk i: fragment reads LOOK_QK k-steps ahead of the MFMAs.
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      {
        const uint32_t tile = tile_address(i);
        uint32_t base[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) base[b] = opaque(tile + qk_base[b]);
        x8 ka0[QK_STEPS], ka1[QK_STEPS];
        auto load = [&](int j) {
          const AFA_LDS uint8_t* q = lds_at<uint8_t>(base[j & 3]) + (j >> 2) * 256;
          ka0[j] = *(const AFA_LDS x8*)q;
          ka1[j] = *(const AFA_LDS x8*)(q + 16 * ROW_BYTES);
        };
#pragma unroll
        for (int j = 0; j < LOOK_QK && j < QK_STEPS; ++j) load(j);
        // Scheduling barriers pin the read distance: left alone, the compiler
        // pulls every read next to its MFMA and each waits a full LDS latency.
#pragma unroll
        for (int j = 0; j < QK_STEPS; ++j) {
          if (j + LOOK_QK < QK_STEPS) load(j + LOOK_QK);
          s0 = B16<DT>::mfma(ka0[j], qf[j], s0);
          s1 = B16<DT>::mfma(ka1[j], qf[j], s1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // Online softmax; the scale is positive, so the chunk max is taken on
      // the raw scores and the scale goes into the exponent's FMA. Only the
      // last chunk holds padding rows.
      const int slot = i & 1;
      float x0[4], x1[4];
      float cmax = -INFINITY;
      // Uniform (readfirstlane): the mask below is then a scalar branch that
      // full chunks skip, not per-element selects on every chunk.
      const int live = __builtin_amdgcn_readfirstlane(placeholder ? 0 : n_rows - list_chunk(i) * CHUNK);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x0[k] = s0[k];
        x1[k] = s1[k];
      }
      if (live < CHUNK) {
        // The empty asm keeps this a branch (it is not speculated into selects).
        __asm__ volatile("");
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int row = sigma(4 * g + k);
          x0[k] = (row < live) ? x0[k] : -INFINITY;
          x1[k] = (16 + row < live) ? x1[k] : -INFINITY;
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) cmax = fmaxf(cmax, fmaxf(x0[k], x1[k]));
      cmax = max_over_lane_groups(cmax);
      const float m_new = fmaxf(m_run, cmax * scale_log2);
      const bool raise = __ballot(m_new > m_run + TAU) != 0ull;
      if (raise) {
        const float alpha = fast_exp2(m_run - m_new);
        l_run *= alpha;
        m_run = m_new;
        if (g == 0) alpha_lds[slot][16 * wave + i16] = alpha;
      }
      if (lane == 0) flag_lds[slot][wave] = raise ? 1 : 0;
      const float neg_m = -m_run;
      float psum = 0.f;
      x8 p8;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float p0 = fast_exp2(__builtin_fmaf(x0[k], scale_log2, neg_m));
        const float p1 = fast_exp2(__builtin_fmaf(x1[k], scale_log2, neg_m));
        psum += p0 + p1;
        p8[k] = (scalar)p0;
        p8[4 + k] = (scalar)p1;
      }
      l_run += psum;
      p_lds[slot][wave][lane] = __builtin_bit_cast(u32x4, p8);
    }
    const float l = sum_over_lane_groups(l_run);
    if (g == 0) {
      // l = 0 only for a split part without rows (its O is 0 and its merge
      // weight l 2^(m - M) is 0); without the sink it has no denominator.
      linv_lds[16 * wave + i16] = l > 0.f ? 1.0f / l : 0.f;
      ml_lds[0][16 * wave + i16] = m_run;
      ml_lds[1][16 * wave + i16] = l;
      if (a.lse != nullptr && !split) a.lse[(size_t)token * a.H + qhead] = lse_of(m_run, l);
    }
    __syncthreads();
  } else {
    // ---- 4b. output wave: O^T[features, heads] += V^T * P^T ------------------
    const int dbase = (wave - NQ) * DPV;
    f32x4 o[NQ][PVT];
#pragma unroll
    for (int ht = 0; ht < NQ; ++ht)
#pragma unroll
      for (int t = 0; t < PVT; ++t) o[ht][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Transposing-read base of 16-feature tile t (t < 8; tile t + 8 is 256
    // bytes further on when the range spans whole swizzle groups).
    constexpr int NB = PVT < 8 ? PVT : 8;
    const int rt = sigma(4 * g + (i16 >> 2));  // chunk row of this lane's read inside a tile
    uint32_t tr_base[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
      tr_base[b] = (uint32_t)(rt * ROW_BYTES + (((dbase / 8 + 2 * b + ((i16 & 3) >> 1)) ^ (rt & 15)) << 4) + (i16 & 1) * 8);

    for (int i = 0; i <= chunks; ++i) {
      step_begin(i);
      if (i == 0) continue;
      const int c = i - 1, slot = c & 1;
      // Rescale flags, P and the first V^T fragments go out together; the
      // flags are waited on first.
      const u32x4 flags = *lds_at<u32x4>(lds_address(flag_lds[slot]));
      x8 pb[NQ];
#pragma unroll
      for (int ht = 0; ht < NQ; ++ht) pb[ht] = __builtin_bit_cast(x8, p_lds[slot][ht][lane]);
      const uint32_t tile = tile_address(c);
      uint32_t vbase[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) vbase[b] = opaque(tile + tr_base[b]);
      x4 vlo[PVT], vhi[PVT];
      auto load_step = [&](int t) {
        const AFA_LDS uint8_t* p = lds_at<uint8_t>(vbase[t % NB]) + (t / NB) * 256;
        vlo[t] = B16<DT>::read_tr((const AFA_LDS void*)p);
        vhi[t] = B16<DT>::read_tr((const AFA_LDS void*)(p + 16 * ROW_BYTES));
      };
#pragma unroll
      for (int t = 0; t < LOOK && t < PVT; ++t) load_step(t);
      // Apply the rescale factors of heads whose running max was raised.
#pragma unroll
      for (int ht = 0; ht < NQ; ++ht) {
        if (__builtin_amdgcn_readfirstlane(flags[ht])) {
          const float alpha = alpha_lds[slot][16 * ht + i16];
#pragma unroll
          for (int t = 0; t < PVT; ++t) o[ht][t] *= alpha;
        }
      }
#pragma unroll
      for (int t = 0; t < PVT; ++t) {
        if (t + LOOK < PVT) load_step(t + LOOK);
        const x8 v = {vlo[t][0], vlo[t][1], vlo[t][2], vlo[t][3], vhi[t][0], vhi[t][1], vhi[t][2], vhi[t][3]};
#pragma unroll
        for (int ht = 0; ht < NQ; ++ht) o[ht][t] = B16<DT>::mfma(v, pb[ht], o[ht][t]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();
    // ---- 5. normalise and store: this lane holds head head0 + 16ht + i16,
    // features dbase + 16t + 4g + i. The KV ring is idle now: each output
    // wave stages its head tiles in its own 16 * DPV * 2 bytes of it.
    static_assert(NP * 16 * DPV * 2 <= NS * CHUNK * ROW_BYTES, "output stage must fit the KV ring");
    if (split) {
      store_record<DT, NQ, NP, DPV>(a, key - S0, part, wave - NQ, o, linv_lds, ml_lds, lane);
      return;
    }
    const uint32_t stage = lds_address(kv_lds[0]) + (uint32_t)((wave - NQ) * 16 * DPV * 2);
    scalar* out0 = (scalar*)a.out + ((size_t)token * a.H + head0) * D + dbase;
#pragma unroll
    for (int ht = 0; ht < NQ; ++ht)
      store_head_tile<DT, DPV, DPV * 2, DPV / 8 - 1, true>(stage, 0u, o[ht], linv_lds[16 * ht + i16],
                                                           out0 + (size_t)16 * ht * D, D, lane);
  }
}

// Stream position: chunk c of work item j (workgroup-local index), whose
// chunks are list chunks first .. first + n - 1 (n = 0: one masked chunk).
struct Cursor {
  int j, c, first, n;
  __device__ __forceinline__ int chunks() const { return n > 0 ? n : 1; }
  __device__ __forceinline__ int list_chunk() const { return n > 0 ? first + c : 0; }
};

// Persistent form for the plan workspace: one workgroup per CU walks its work
// items worker, worker + G, ... (G workgroups; an item is one (token, BM-head
// tile) key) as ONE continuous chunk stream, so an item boundary costs no
// pipeline drain and no dependent global round trip.
//  - the KV ring of NS tiles, P slots and step parities run on across items;
//    output waves fetch KV rows AHEAD = NS - 2 chunks ahead of the score waves
//    (3 tiles: one chunk in flight, for rows re-read from the caches; 4: two,
//    for rows streamed from HBM);
//  - output waves copy the row list (and count) of item j + LISTS - 1 when
//    item j starts, into a ring of LISTS LDS lists;
//  - score waves load Q and the sinks of item j + 1 into registers when item j
//    starts and issue no other vector memory loads, so those loads have a
//    whole item to land (vector loads of a wave complete in issue order, so a
//    score-wave KV fetch would wait for them);
//  - each item's running max starts at its sinks (one lane group counts the
//    sink's e^(sink - m)), its output accumulators are cleared on its first PV
//    step, and its denominator travels through LDS slot item & 1.
// The first item's Q goes through LDS as in sparse_mla_kernel.
// STREAM: KV row loads, next-item Q loads and O stores are non-temporal, for
// calls whose requests have few query tokens (batched decode: rows shared by
// few tokens); prefill keeps ordinary accesses, its consecutive tokens
// sharing rows through the L2.
template <int DT, int D, int NQ, int NP, int NS, bool CLAMP, bool STREAM = false>
__global__ __launch_bounds__((NQ + NP) * 64) void sparse_mla_persistent_kernel(SparseArgs a) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x8 x8;
  typedef typename B16<DT>::x4 x4;
  constexpr int NW = NQ + NP;
  constexpr int BMH = 16 * NQ;
  constexpr int UNITS = D / 8;
  constexpr int ROW_BYTES = D * 2;
  constexpr int QK_STEPS = D / 32;
  constexpr int DPV = D / NP;
  constexpr int PVT = DPV / 16;
  constexpr int NO = NP * 64;                  // fetching threads (output waves)
  constexpr int PIECES = CHUNK * UNITS / NO;   // 16-byte loads per output thread per chunk
  constexpr int AHEAD = NS - 2;                // chunks fetched ahead of the score waves
  constexpr int LISTS = AHEAD + 3;             // row-list ring (items j - 1 .. j + AHEAD + 1 in use)
  static_assert(NS == 3 || NS == 4, "KV ring of 3 or 4 tiles");
  static_assert(CHUNK * UNITS % NO == 0, "chunk must split evenly over the output waves");
  static_assert(UNITS >= 16, "swizzle needs at least 16 units per row");
  static_assert(DPV % 16 == 0 && (PVT <= 8 || (DPV / 8) % 16 == 0), "output feature range");
  static_assert(NQ == NP && NQ <= 4, "one score and one output wave per SIMD");

  __shared__ __attribute__((aligned(16))) uint8_t kv_lds[NS][CHUNK * ROW_BYTES];
  __shared__ __attribute__((aligned(16))) u32x4 p_lds[2][NQ][64];
  __shared__ float alpha_lds[2][BMH];
  __shared__ __attribute__((aligned(16))) int flag_lds[2][4];
  __shared__ float l_lds[2][BMH];  // item parity: softmax denominator per head
  __shared__ __attribute__((aligned(16))) int count_lds[LISTS];
  extern __shared__ __attribute__((aligned(16))) uint32_t lists[];  // [LISTS][list_pad]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 4, i16 = lane & 15;
  const bool scorer = wave < NQ;
  const int head_tiles = a.H / a.BM;
  const int n_items = a.T * head_tiles;
  const int G = (int)gridDim.x;
  const int worker = (int)xcd_contiguous(blockIdx.x, gridDim.x);
  const int J = (n_items - worker + G - 1) / G;  // items of this workgroup (>= 1: G <= n_items)
  auto item_key = [&](int j) { return worker + j * G; };
  auto item_token = [&](int j) { return item_key(j) / head_tiles; };
  auto item_head0 = [&](int j) { return (item_key(j) % head_tiles) * a.BM; };
  const uint32_t list_base = lds_address(lists);
  auto list_address = [&](int j) { return list_base + (uint32_t)((j % LISTS) * a.list_pad) * 4u; };
  // Selected rows of item j, at most the list capacity (a plan of other sizes
  // cannot index past the LDS row list).
  auto count_of = [&](int j) { return min(count_lds[j % LISTS], a.list_pad); };
  auto start = [&](Cursor& k, int j) {
    const PartRange r = part_range(count_of(j), 0, 1);
    k.j = j;
    k.c = 0;
    k.first = r.first;
    k.n = r.n;
  };
  auto advance = [&](Cursor& k) -> bool {  // false at the end of the stream (k.j becomes J)
    if (++k.c < k.chunks()) return true;
    if (k.j + 1 >= J) {
      k.j = J;
      return false;
    }
    start(k, k.j + 1);
    return true;
  };

  // Row list and count of item j: output waves split the 1 KiB units.
  auto copy_list = [&](int j) {
    const int token = item_token(j);
    const uint32_t* src = a.plan_rows + (size_t)token * a.list_pad;
    const uint32_t dst = list_address(j);
    if (wave == NQ && lane == 0)
      __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
                       :: "s"(lds_address(&count_lds[j % LISTS])), "v"(0u), "s"(a.plan_count + token) : "memory");
    for (int u = wave - NQ; u < a.list_pad / 256; u += NP)
      __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                       :: "s"(dst + (uint32_t)u * 1024u), "v"((uint32_t)lane * 16u), "s"(src + u * 256) : "memory");
  };

  // ---- prologue: lists of items 0..LISTS-2, Q of item 0 through the last two ring tiles ----
  const uint32_t q_lds = lds_address(kv_lds[NS - 2]);
  constexpr int Q_LOADS = BMH * ROW_BYTES / 1024;
  static_assert(BMH * ROW_BYTES <= 2 * CHUNK * ROW_BYTES, "Q tile must fit two ring tiles");
  static_assert(Q_LOADS % NW == 0, "Q tile must split evenly over the waves");
  constexpr int Q_LOADS_PER_WAVE = Q_LOADS / NW;
  if (!scorer)
    for (int j = 0; j < J && j < LISTS - 1; ++j) copy_list(j);
  {
    const char* q_src = (const char*)a.q + ((size_t)item_token(0) * a.H + item_head0(0)) * ROW_BYTES;
#pragma unroll
    for (int k0 = 0; k0 < Q_LOADS; k0 += NW) {
      const int k = k0 + wave;
      const int pos = k * 64 + lane;
      const int r = pos / UNITS, u = pos % UNITS;
      const uint32_t off = (uint32_t)(r * ROW_BYTES + ((u ^ (r & 15)) << 4));
      __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                       :: "s"(q_lds + (uint32_t)k * 1024u), "v"(off), "s"(q_src) : "memory");
    }
  }
  // Lists landed (Q may still be in flight).
  __builtin_amdgcn_s_waitcnt(0x0F70 | (Q_LOADS_PER_WAVE & 15) | ((Q_LOADS_PER_WAVE >> 4) << 14));
  block_barrier();

  // ---- KV fetch by the output waves ------------------------------------------
  constexpr bool ROW_LOADS = (UNITS == 64);
  const char* ori = (const char*)a.ori_kv;
  const char* cmp = (const char*)a.cmp_kv;
  const uint32_t kv_base = lds_address(kv_lds[0]);
  auto tile_address = [&](int s) {
    return opaque_uniform(kv_base + (uint32_t)(s % NS) * (CHUNK * ROW_BYTES));
  };
  const int ow = wave - NQ;  // output wave index (fetch role)
  uint32_t unit_offset[PIECES];
#pragma unroll
  for (int p = 0; p < PIECES; ++p) unit_offset[p] = (uint32_t)((lane ^ ((ow * PIECES + p) & 15)) << 4);
  // Entries of the next chunk to fetch (ROW_LOADS), read one fetch ahead.
  uint32_t entry_next[PIECES];
  auto read_entries = [&](const Cursor& k) {
    const AFA_LDS uint32_t* l = lds_at<uint32_t>(list_address(k.j));
#pragma unroll
    for (int p = 0; p < PIECES; ++p) entry_next[p] = l[k.list_chunk() * CHUNK + ow * PIECES + p];
  };
  // CLAMP (the planned entry point, whose plan is a workspace the caller
  // hands over): each row is clamped to its cache, so an entry that is not
  // from a plan of these sizes reads a wrong row, never memory outside the
  // caches. Plans written by this library's plan kernel need no clamp (two
  // more scalar operations per row cost ~3.5% on prefill).
  const uint32_t ori_last = (uint32_t)(a.ori_blocks * a.PAGE - 1);
  const uint32_t cmp_last = (uint32_t)(a.cmp_blocks * (a.PAGE / a.RATIO) - 1);
  auto row_of = [&](uint32_t e) {
    const bool c = (e & CMP_BIT) != 0u;
    const uint32_t r = e & ~CMP_BIT;
    return (c ? cmp : ori) + (size_t)(CLAMP ? min(r, c ? cmp_last : ori_last) : r) * ROW_BYTES;
  };
  // The chunk at cursor k into ring tile s % NS (ROW_LOADS: entries already read).
  auto fetch = [&](int s, const Cursor& k) {
    const uint32_t tile = tile_address(s);
    if constexpr (ROW_LOADS) {
#pragma unroll
      for (int p = 0; p < PIECES; ++p) {
        const int r = ow * PIECES + p;
        const uint32_t e = __builtin_amdgcn_readfirstlane(entry_next[p]);
        const char* row = row_of(e);
        if constexpr (STREAM)
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                           :: "s"(tile + (uint32_t)(r * ROW_BYTES)), "v"(unit_offset[p]), "s"(row) : "memory");
        else
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                           :: "s"(tile + (uint32_t)(r * ROW_BYTES)), "v"(unit_offset[p]), "s"(row) : "memory");
      }
    } else {
      const AFA_LDS uint32_t* l = lds_at<uint32_t>(list_address(k.j));
      const int otid = tid - NQ * 64;
#pragma unroll
      for (int p = 0; p < PIECES; ++p) {
        const int flat = otid + p * NO;
        const int r = flat / UNITS, upos = flat % UNITS;
        const uint32_t e = l[k.list_chunk() * CHUNK + r];
        const char* src = row_of(e) + ((upos ^ (r & 15)) << 4);
        if constexpr (STREAM)
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt"
                           :: "s"(tile + (uint32_t)((ow * 64 + p * NO) * 16)), "v"(src) : "memory");
        else
          __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                           :: "s"(tile + (uint32_t)((ow * 64 + p * NO) * 16)), "v"(src) : "memory");
      }
    }
  };

  // ---- stream cursors (uniform and identical in every wave) ------------------
  // The score cursor; the output waves' fetch cursor runs AHEAD chunks ahead.
  Cursor cur;
  start(cur, 0);
  Cursor fcur = cur;
  bool fvalid = true;         // fcur is inside the stream
  bool ahead_loaded = false;  // the last fetch issued is a chunk after the next one consumed
  if (!scorer) {
    if constexpr (ROW_LOADS) read_entries(fcur);
    int issued = 0;
#pragma unroll
    for (int k = 0; k < AHEAD; ++k) {
      if (fvalid) {
        fetch(k, fcur);
        ++issued;
        fvalid = advance(fcur);
        if (ROW_LOADS && fvalid) read_entries(fcur);
      }
    }
    ahead_loaded = issued > 1;
    // Q has landed once at most the loads of the prologue fetches are in flight.
    if (issued > 1)
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * PIECES) & 15) | (((2 * PIECES) >> 4) << 14));
    else
      __builtin_amdgcn_s_waitcnt(0x0F70 | (PIECES & 15) | ((PIECES >> 4) << 14));
  } else {
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
  block_barrier();

  if (scorer) {
    // ---- score waves ------------------------------------------------------------
    const float scale_log2 = a.scale * LOG2E;
    const int ra = sigma(i16);
    uint32_t qk_base[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) qk_base[b] = (uint32_t)(ra * ROW_BYTES + (((4 * b + g) ^ (ra & 15)) << 4));
    x8 qf[QK_STEPS], qf_next[QK_STEPS];
    {
      const int r = 16 * wave + i16;
#pragma unroll
      for (int k = 0; k < QK_STEPS; ++k)
        qf[k] = *lds_at<x8>(q_lds + (uint32_t)(r * ROW_BYTES + (((4 * k + g) ^ (r & 15)) << 4)));
    }
    float sink = a.sinks[item_head0(0) + 16 * wave + i16] * LOG2E, sink_next = 0.f;
    float m_run = 0.f, l_run = 0.f;
    for (int s = 0;; ++s) {
      if (cur.j >= J) {  // stream done: one more barrier for the last PV, then leave
        block_barrier();
        break;
      }
      block_barrier();
      if (cur.c == 0) {
        if (cur.j > 0) {
#pragma unroll
          for (int k = 0; k < QK_STEPS; ++k) qf[k] = qf_next[k];
          sink = sink_next * LOG2E;
        }
        m_run = sink;
        l_run = g == 0 ? 1.0f : 0.0f;  // e^(sink - m) counted once per head
        if (cur.j + 1 < J) {
          const int head = item_head0(cur.j + 1) + 16 * wave + i16;
          const scalar* q_row = (const scalar*)a.q + ((size_t)item_token(cur.j + 1) * a.H + head) * D + 8 * g;
#pragma unroll
          for (int k = 0; k < QK_STEPS; ++k) {
            if constexpr (STREAM)
              qf_next[k] = __builtin_nontemporal_load((const x8*)(q_row + 32 * k));
            else
              qf_next[k] = *(const x8*)(q_row + 32 * k);
          }
          // Used (scaled) only when the next item starts: vector loads retire
          // in order, so consuming it here would wait for all of Q's loads,
          // a full HBM round trip at every item start.
          sink_next = a.sinks[head];
        }
      }
      // S^T of this chunk: fragment reads LOOK_QK k-steps ahead of the MFMAs.
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      {
        const uint32_t tile = tile_address(s);
        uint32_t base[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) base[b] = opaque(tile + qk_base[b]);
        x8 ka0[QK_STEPS], ka1[QK_STEPS];
        auto load = [&](int k) {
          const AFA_LDS uint8_t* q = lds_at<uint8_t>(base[k & 3]) + (k >> 2) * 256;
          ka0[k] = *(const AFA_LDS x8*)q;
          ka1[k] = *(const AFA_LDS x8*)(q + 16 * ROW_BYTES);
        };
#pragma unroll
        for (int k = 0; k < LOOK_QK && k < QK_STEPS; ++k) load(k);
#pragma unroll
        for (int k = 0; k < QK_STEPS; ++k) {
          if (k + LOOK_QK < QK_STEPS) load(k + LOOK_QK);
          s0 = B16<DT>::mfma(ka0[k], qf[k], s0);
          s1 = B16<DT>::mfma(ka1[k], qf[k], s1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      const int slot = s & 1;
      float x0[4], x1[4];
      float cmax = -INFINITY;
      // Rows of this chunk that hold selected entries (<= 0: masked placeholder).
      // Uniform (readfirstlane): the mask below is then a scalar branch that
      // full chunks skip, not per-element selects on every chunk.
      const int live =
          __builtin_amdgcn_readfirstlane(cur.n > 0 ? count_of(cur.j) - (cur.first + cur.c) * CHUNK : 0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x0[k] = s0[k];
        x1[k] = s1[k];
      }
      if (live < CHUNK) {
        // The empty asm keeps this a branch (it is not speculated into selects).
        __asm__ volatile("");
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int row = sigma(4 * g + k);
          x0[k] = (row < live) ? x0[k] : -INFINITY;
          x1[k] = (16 + row < live) ? x1[k] : -INFINITY;
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) cmax = fmaxf(cmax, fmaxf(x0[k], x1[k]));
      cmax = max_over_lane_groups(cmax);
      const float m_new = fmaxf(m_run, cmax * scale_log2);
      const bool raise = __ballot(m_new > m_run + TAU) != 0ull;
      if (raise) {
        const float alpha = fast_exp2(m_run - m_new);
        l_run *= alpha;
        m_run = m_new;
        if (g == 0) alpha_lds[slot][16 * wave + i16] = alpha;
      }
      if (lane == 0) flag_lds[slot][wave] = raise ? 1 : 0;
      const float neg_m = -m_run;
      float psum = 0.f;
      x8 p8;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float p0 = fast_exp2(__builtin_fmaf(x0[k], scale_log2, neg_m));
        const float p1 = fast_exp2(__builtin_fmaf(x1[k], scale_log2, neg_m));
        psum += p0 + p1;
        p8[k] = (scalar)p0;
        p8[4 + k] = (scalar)p1;
      }
      l_run += psum;
      p_lds[slot][wave][lane] = __builtin_bit_cast(u32x4, p8);
      if (cur.c == cur.chunks() - 1) {
        const float l = sum_over_lane_groups(l_run);
        if (g == 0) {
          l_lds[cur.j & 1][16 * wave + i16] = l;
          if (a.lse != nullptr)
            a.lse[(size_t)item_token(cur.j) * a.H + item_head0(cur.j) + 16 * wave + i16] = lse_of(m_run, l);
        }
      }
      advance(cur);
    }
  } else {
    // ---- output waves: fetch, then O^T[features, heads] += V^T * P^T ----------
    // Their step (fetch issue, then PV) is the longer one: a higher wave
    // priority lets their instructions, MFMAs included, win the arbitration
    // against the score wave of the same SIMD (prefill Q8K about 3% faster).
    __builtin_amdgcn_s_setprio(2);
    const int dbase = ow * DPV;
    f32x4 o[NQ][PVT];
    constexpr int NB = PVT < 8 ? PVT : 8;
    const int rt = sigma(4 * g + (i16 >> 2));
    uint32_t tr_base[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
      tr_base[b] = (uint32_t)(rt * ROW_BYTES + (((dbase / 8 + 2 * b + ((i16 & 3) >> 1)) ^ (rt & 15)) << 4) + (i16 & 1) * 8);

    // Output of item j: this lane holds heads head0 + 16ht + i16, features
    // dbase + 16t + 4g + i. The stores are staged (store_head_tile) in this
    // wave's own feature units of rows 0..15 of the ring tile whose PV just
    // ended: during this step only output waves read that tile, each its own
    // feature units (the tile swizzle XORs the unit with row & 15, which keeps
    // it among the wave's units, or in row-by-row groups of as many units), and
    // the fetch that refills the tile is issued after the next barrier.
    static_assert(CHUNK >= 16, "a head tile's stage rows fit a ring tile");
    auto finish = [&](int j, uint32_t tile) {
      const int key = item_key(j), par = j & 1;
      const int token = key / head_tiles, head0 = (key % head_tiles) * a.BM;
      scalar* out0 = (scalar*)a.out + ((size_t)token * a.H + head0) * D + dbase;
#pragma unroll
      for (int ht = 0; ht < NQ; ++ht) {
        const float inv = 1.0f / l_lds[par][16 * ht + i16];
        store_head_tile<DT, DPV, ROW_BYTES, 15, STREAM>(tile, (uint32_t)(dbase / 8), o[ht], inv, out0 + (size_t)16 * ht * D,
                                                D, lane);
      }
    };

    Cursor ocur = cur;   // output cursor: the score cursor of the previous step
    bool ovalid = false;
    bool stored = false;  // the previous step issued global stores
    for (int s = 0;; ++s) {
      const bool score_active = cur.j < J;
      if (!score_active && !ovalid) break;
      // KV(s) has landed once at most the younger fetch batch is in flight
      // (only loads are in flight then). After output stores the wait is for
      // everything (vmcnt(0)): a partial wait is never taken behind stores.
      if (stored || !ahead_loaded)
        wait_vmcnt<0>();
      else
        wait_vmcnt<PIECES>();
      block_barrier();
      stored = false;
      ahead_loaded = false;
      if (score_active) {
        if (cur.c == 0 && cur.j + LISTS - 1 < J) copy_list(cur.j + LISTS - 1);
        if (fvalid) {
          fetch(s + AHEAD, fcur);
          fvalid = advance(fcur);
          if (ROW_LOADS && fvalid) read_entries(fcur);
          ahead_loaded = AHEAD > 1;
        }
      }
      if (ovalid) {
        const int slot = (s - 1) & 1;
        if (ocur.c == 0) {
#pragma unroll
          for (int ht = 0; ht < NQ; ++ht)
#pragma unroll
            for (int t = 0; t < PVT; ++t) o[ht][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        const u32x4 flags = *lds_at<u32x4>(lds_address(flag_lds[slot]));
        x8 pb[NQ];
#pragma unroll
        for (int ht = 0; ht < NQ; ++ht) pb[ht] = __builtin_bit_cast(x8, p_lds[slot][ht][lane]);
        const uint32_t tile = tile_address(s - 1);
        uint32_t vbase[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) vbase[b] = opaque(tile + tr_base[b]);
        x4 vlo[PVT], vhi[PVT];
        auto load_step = [&](int t) {
          const AFA_LDS uint8_t* p = lds_at<uint8_t>(vbase[t % NB]) + (t / NB) * 256;
          vlo[t] = B16<DT>::read_tr((const AFA_LDS void*)p);
          vhi[t] = B16<DT>::read_tr((const AFA_LDS void*)(p + 16 * ROW_BYTES));
        };
#pragma unroll
        for (int t = 0; t < LOOK && t < PVT; ++t) load_step(t);
#pragma unroll
        for (int ht = 0; ht < NQ; ++ht) {
          if (__builtin_amdgcn_readfirstlane(flags[ht])) {
            const float alpha = alpha_lds[slot][16 * ht + i16];
#pragma unroll
            for (int t = 0; t < PVT; ++t) o[ht][t] *= alpha;
          }
        }
#pragma unroll
        for (int t = 0; t < PVT; ++t) {
          if (t + LOOK < PVT) load_step(t + LOOK);
          const x8 v = {vlo[t][0], vlo[t][1], vlo[t][2], vlo[t][3], vhi[t][0], vhi[t][1], vhi[t][2], vhi[t][3]};
#pragma unroll
          for (int ht = 0; ht < NQ; ++ht) o[ht][t] = B16<DT>::mfma(v, pb[ht], o[ht][t]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (ocur.c == ocur.chunks() - 1) {
          finish(ocur.j, tile);
          stored = true;
        }
      }
      if (score_active) {
        ocur = cur;
        ovalid = true;
        advance(cur);
      } else {
        ovalid = false;
      }
    }
  }
}

// Merge of split work items (records: store_record). One workgroup per
// (split key, output wave ow, 16-head tile) slice, each thread issuing all of
// its parts' loads at once, combines the parts in part order (deterministic):
// with M = max_p m_p and w_p = 2^(m_p - M) l_p (part p's denominator relative
// to M), O = sum_p w_p O_p / sum_p w_p, O_p the part's normalised output: the
// online-softmax merge of attention.py:398-525's running max and denominator
// over disjoint row sets (the sink's term is in part 0's denominator).
template <int D, int NP>
constexpr int merge_threads() {  // threads per 16-head slice: at most 256
  return (D / NP / 16) * 64 < 256 ? (D / NP / 16) * 64 : 256;
}
template <int DT, int D, int NQ, int NP>
__global__ __launch_bounds__((merge_threads<D, NP>())) void sparse_merge_kernel(SparseArgs a) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x4 x4;
  constexpr int BMH = 16 * NQ;
  constexpr int DPV = D / NP;
  constexpr int PVT = DPV / 16;
  constexpr int MT = merge_threads<D, NP>();
  constexpr int PER = PVT * 64 / MT;  // x4 of a 16-head slice per thread
  static_assert(PVT * 64 % MT == 0 && PER >= 1 && PER <= 4, "slice must split evenly over the threads");
  constexpr size_t REC = record_bytes<DT>(BMH, DPV);
  const int slice = (int)blockIdx.x % (NP * NQ), split_key = (int)blockIdx.x / (NP * NQ);
  const int ow = slice / NQ, ht = slice % NQ;
  const int head_tiles = a.H / a.BM;
  const int key = a.split_from + split_key;
  const int token = key / head_tiles, head0 = (key % head_tiles) * a.BM;
  const int P = a.parts;
  // Thread tid holds x4 number ht * PVT * 64 + k * MT + tid of the slice:
  // tile t = (k * MT + tid) / 64, lane = tid % 64.
  const int lane = threadIdx.x & 63, i16 = lane & 15, g = lane >> 4;
  const int h = 16 * ht + i16;
  float mq[MAX_PARTS], lq[MAX_PARTS];
  x4 oq[MAX_PARTS][PER];
#pragma unroll
  for (int q = 0; q < MAX_PARTS; ++q) {
    if (q < P) {
      const char* rec = (const char*)a.partials + (((size_t)split_key * P + q) * NP + ow) * REC;
      const float* stats = (const float*)(rec + (size_t)BMH * DPV * sizeof(scalar));
      mq[q] = stats[h];
      lq[q] = stats[BMH + h];
#pragma unroll
      for (int k = 0; k < PER; ++k)
        oq[q][k] = *(const x4*)(rec + (size_t)(ht * PVT * 64 + k * MT + threadIdx.x) * sizeof(x4));
    }
  }
  float M = -INFINITY;
#pragma unroll
  for (int q = 0; q < MAX_PARTS; ++q)
    if (q < P) M = fmaxf(M, mq[q]);
  float L = 0.f;
  f32x4 acc[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < MAX_PARTS; ++q) {
    if (q < P) {
      const float w = fast_exp2(mq[q] - M) * lq[q];
      L += w;
#pragma unroll
      for (int k = 0; k < PER; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[k][e] += (float)oq[q][k][e] * w;
    }
  }
  const float inv = 1.0f / L;
  if (a.lse != nullptr && ow == 0 && threadIdx.x < 16) a.lse[(size_t)token * a.H + head0 + h] = lse_of(M, L);
  scalar* out_row = (scalar*)a.out + ((size_t)token * a.H + head0 + h) * D + ow * DPV + 4 * g;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int t = (k * MT + (int)threadIdx.x) / 64;
    x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (scalar)(acc[k][e] * inv);
    *(x4*)(out_row + 16 * t) = v;
  }
}

// Gather image: one block per token, slot-major copy of the selected rows
// through the fused kernel's slot resolution (resolve_slot, row_pointer).
template <int DT>
__global__ __launch_bounds__(256) void sparse_gather_kernel(SparseArgs a, void* kv_out,
                                                            float* bias_out) {
  typedef typename B16<DT>::scalar scalar;
  const int token = blockIdx.x;
  const Geometry geo = token_geometry(a, token, request_by_search(a, token));
  const int slots = a.WINDOW + geo.count_cmp;
  const int units = a.D / 8;
  for (int s = 0; s < a.S; ++s) {
    uint32_t entry = 0;
    const bool valid = s < slots && resolve_slot(a, geo, token, s, entry);
    u32x4* dst = (u32x4*)((scalar*)kv_out + ((size_t)token * a.S + s) * a.D);
    const scalar* src = valid ? row_pointer<scalar>(a, entry) : nullptr;
    for (int u = threadIdx.x; u < units; u += blockDim.x)
      dst[u] = valid ? *(const u32x4*)(src + u * 8) : u32x4{0u, 0u, 0u, 0u};
    if (threadIdx.x == 0) bias_out[(size_t)token * a.S + s] = valid ? 0.0f : -INFINITY;
  }
}

// Gather probe, a measurement kernel with no counterpart on the attention path
// (the reference's standalone gather micro-benchmark is
// benchmarks/attention/gather_dma.py): streams the row lists of a plan
// workspace through LDS the way the attention kernels move KV rows
// (load-to-LDS, one wave load per 1 KiB row, the same XOR swizzle), in
// 16-row chunks with DEPTH chunks in flight per workgroup, and no compute. It
// measures the HBM rate the sparse access pattern itself reaches at a given
// depth. Each workgroup takes up to PROBE_ITEMS items: items worker,
// worker + G, ... (interleaved, as the persistent kernel), or, when balanced,
// an equal range of the flat chunk stream of all items (every item streaming
// as many chunks as item 0). One dword of every streamed row is read back from
// LDS and summed per thread into sums[block][16], so the data can be checked.
constexpr int PROBE_ROWS = 16;   // rows per probe chunk
constexpr int PROBE_ITEMS = 4;   // most items one probe workgroup streams
template <int DEPTH>
__global__ __launch_bounds__(256) void gather_probe_kernel(const char* ori, const char* cmp, const int32_t* counts,
                                                           const uint32_t* lists, int list_pad, int n_items,
                                                           int balanced, uint32_t* sums) {
  constexpr int NT = DEPTH + 1;  // ring tiles: the tile read at step s is never the one being filled
  constexpr int ROW = 1024, PER_WAVE = PROBE_ROWS / 4;
  __shared__ __attribute__((aligned(16))) uint8_t tiles[NT][PROBE_ROWS * ROW];
  extern __shared__ __attribute__((aligned(16))) uint32_t probe_lists[];  // [PROBE_ITEMS][list_pad]
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int G = (int)gridDim.x, worker = (int)xcd_contiguous(blockIdx.x, gridDim.x);
  auto chunks_of = [&](int item) { const int n = counts[item]; return n > 0 ? (n + PROBE_ROWS - 1) / PROBE_ROWS : 1; };
  // This workgroup's items and the chunk range of each.
  int item[PROBE_ITEMS], first[PROBE_ITEMS], nch[PROBE_ITEMS], J = 0;
  if (balanced) {
    const int per = chunks_of(0);
    const long total = (long)n_items * per;
    const long f0 = total * worker / G, f1 = total * (worker + 1) / G;
    for (long f = f0; f < f1 && J < PROBE_ITEMS;) {
      const int it = (int)(f / per), c0 = (int)(f % per);
      const int c1 = (int)min((long)per, f1 - (long)it * per);
      item[J] = it; first[J] = c0; nch[J] = c1 - c0; ++J;
      f = (long)it * per + c1;
    }
  } else {
    for (int it = worker; it < n_items && J < PROBE_ITEMS; it += G) {
      item[J] = it; first[J] = 0; nch[J] = chunks_of(it); ++J;
    }
  }
  // Lists of all items to LDS, one round trip.
  for (int j = 0; j < J; ++j)
    for (int u = wave; u < list_pad / 256; u += 4)
      __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                       :: "s"(lds_address(probe_lists) + (uint32_t)(j * list_pad + u * 256) * 4u),
                          "v"((uint32_t)lane * 16u), "s"(lists + (size_t)item[j] * list_pad + u * 256) : "memory");
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  block_barrier();
  int total = 0, last[PROBE_ITEMS];
  for (int j = 0; j < J; ++j) {
    total += nch[j];
    last[j] = chunks_of(item[j]) - 1;  // the plan holds whole chunks up to here
  }
  auto issue = [&](int s) {
    int j = 0, c = s;
    while (j + 1 < J && c >= nch[j]) c -= nch[j++];
    // Balanced ranges assume item 0's chunk count for every item; an item
    // with fewer listed chunks re-reads its last one, never unwritten entries.
    c = min(c + first[j], last[j]);
    const uint32_t tile = lds_address(tiles[s % NT]);
#pragma unroll
    for (int p = 0; p < PER_WAVE; ++p) {
      const int r = wave * PER_WAVE + p;
      const uint32_t e = __builtin_amdgcn_readfirstlane(probe_lists[j * list_pad + c * PROBE_ROWS + r]);
      const char* row = ((e & CMP_BIT) ? cmp : ori) + (size_t)(e & ~CMP_BIT) * ROW;
      __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                       :: "s"(tile + (uint32_t)(r * ROW)), "v"((uint32_t)((lane ^ (r & 15)) << 4)), "s"(row) : "memory");
    }
  };
  uint32_t acc = 0;
  for (int s = 0; s < DEPTH && s < total; ++s) issue(s);
  for (int s = 0; s < total; ++s) {
    if (s + DEPTH - 1 < total)
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((PER_WAVE * (DEPTH - 1)) & 15) | (((PER_WAVE * (DEPTH - 1)) >> 4) << 14));
    else
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    block_barrier();
    if (tid < PROBE_ROWS)  // unit 0 of row tid sits at position tid & 15
      acc += *lds_at<uint32_t>(lds_address(tiles[s % NT]) + (uint32_t)(tid * ROW + ((tid & 15) << 4)));
    if (s + DEPTH < total) issue(s + DEPTH);
  }
  if (tid < PROBE_ROWS) sums[(size_t)blockIdx.x * PROBE_ROWS + tid] = acc;
}

}  // namespace afa

using namespace afa;

static int check_sparse(const SparseMlaParams* p) {
  if (!p) return AFA_E_NULL;
  if (p->dtype != AFA_DTYPE_BF16 && p->dtype != AFA_DTYPE_F16) return AFA_E_DTYPE;
  if (p->B <= 0 || p->T <= 0 || p->H <= 0) return AFA_E_SHAPE;
  if (p->D != 128 && p->D != 256 && p->D != 512) return AFA_E_SHAPE;
  if (p->BM != 32 && p->BM != 64) return AFA_E_SHAPE;
  if (p->H % p->BM) return AFA_E_SHAPE;
  if (p->PAGE <= 0 || (p->RATIO != 1 && p->RATIO != 2) || p->PAGE % p->RATIO) return AFA_E_SHAPE;
  if (p->MAX_SEQ <= 0 || p->MAX_SEQ % p->PAGE) return AFA_E_SHAPE;
  if (p->WINDOW < 0 || p->WINDOW > 4096 || p->TOPK < 0 || p->TOPK > 8192) return AFA_E_SHAPE;
  // At least one gather slot: the row lists (workspace and LDS) are sized by
  // WINDOW + TOPK, and every token streams at least one chunk.
  if (p->WINDOW + p->TOPK < 1) return AFA_E_SHAPE;
  if (p->S < p->WINDOW + p->TOPK) return AFA_E_SHAPE;
  if (p->ORI_BLOCKS <= 0 || p->CMP_BLOCKS <= 0) return AFA_E_SHAPE;
  if ((int64_t)p->ORI_BLOCKS * p->PAGE >= (int64_t)CMP_BIT) return AFA_E_SHAPE;
  if ((int64_t)p->CMP_BLOCKS * (p->PAGE / p->RATIO) >= (int64_t)CMP_BIT) return AFA_E_SHAPE;
  if (!(p->scale > 0.0f)) return AFA_E_SHAPE;
  if (p->parts < 0 || p->parts > MAX_PARTS) return AFA_E_SHAPE;
  if (p->ring != 0 && p->ring != 3 && p->ring != 4) return AFA_E_SHAPE;
  if ((int64_t)p->T * (p->H / p->BM) * MAX_PARTS > 0x7fffffffLL) return AFA_E_SHAPE;
  return AFA_OK;
}

// Split of the (token, BM-head tile) keys of short streams (at most one full
// round of 256 keys; a fixed model of MI355X's 256 compute units keeps the
// workspace size a function of the sizes alone). With r keys beyond the full
// rounds, the last round keeps only r CUs busy for a whole key's chunks;
// splitting those keys into P parts (r P <= 256) shortens that round, and the
// merge kernel then combines the parts' records. Costs are in chunk steps of a
// fully loaded GPU (256 CUs streaming 32-row chunks, HBM-bound: ~1.4 us at
// D = 512, measured with per-workgroup real-time stamps on decode): a round of
// n streams of c chunks costs SPLIT_SETUP (row resolution and Q) plus
// c * max(SPLIT_LATENCY, n / 256) (fewer streams run latency-bound, not
// faster); the merge costs its launch gap plus its traffic (records written and
// read back, output written) at the loaded rate of 256 chunks per step. The
// cheapest P is taken if it beats the whole last round: decode B1..B16 x 6 and
// B48 x 6 split; B64 x 6 (128 keys beyond one round: 10 loaded steps plus a
// merge of 7 against 20 latency-bound ones of 0.7) does not, nor does anything
// with two or more full rounds (those run on the persistent kernel).
// parts = 1 never splits; parts > 1 splits every key into that many parts.
struct Split {
  int parts;           // parts of each split key (1: nothing split)
  int64_t split_from;  // first split key
};
constexpr int64_t SPLIT_MODEL_CUS = 256;
constexpr double SPLIT_SETUP = 3.5, SPLIT_LATENCY = 0.7, MERGE_GAP = 2.0;
static int64_t record_bytes_per_part(const SparseMlaParams* p) {
  // BM heads x D features of the storage dtype, plus FP32 (max, denominator)
  // per head and output wave (BM / 16 output waves).
  return 2LL * p->BM * p->D + (int64_t)p->BM * p->BM / 2;
}
static Split choose_split(const SparseMlaParams* p) {
  const int64_t tiles = (int64_t)p->T * (p->H / p->BM);
  if (p->parts == 1) return Split{1, tiles};
  if (p->parts > 1) return Split{p->parts, 0};
  const int64_t nch = std::max<int64_t>(1, (p->WINDOW + p->TOPK + CHUNK - 1) / CHUNK);
  const int64_t rounds = tiles / SPLIT_MODEL_CUS, rest = tiles % SPLIT_MODEL_CUS;
  if (rest == 0 || rounds > 1) return Split{1, tiles};
  const double cus = (double)SPLIT_MODEL_CUS;
  auto round_cost = [&](int64_t n, int64_t c) { return SPLIT_SETUP + c * std::max(SPLIT_LATENCY, n / cus); };
  const double step_bytes = cus * CHUNK * p->D * 2.0;
  Split best{1, tiles};
  double best_cost = round_cost(rest, nch);
  const int64_t max_parts = std::min<int64_t>(std::min<int64_t>(MAX_PARTS, SPLIT_MODEL_CUS / rest), nch);
  for (int64_t parts = 2; parts <= max_parts; ++parts) {
    const double traffic = (double)rest * (2.0 * parts * record_bytes_per_part(p) + 2.0 * p->BM * p->D);
    const double cost = round_cost(rest * parts, (nch + parts - 1) / parts) + MERGE_GAP + traffic / step_bytes;
    if (cost < best_cost) {
      best_cost = cost;
      best = Split{(int)parts, rounds * SPLIT_MODEL_CUS};
    }
  }
  return best;
}

// MI355X's Infinity Cache (the memory-side cache in front of HBM). Caches
// larger than it stream mostly from HBM, where two chunks in flight (a 4-tile
// ring) pay: decode B86 / B128 / B170 / B256 x 6 at 128K 9% / 2.4% / 4.3% /
// 5.3% faster, B128 x 6 at 32K 2.8%, a 4 x 2K prefill at 128K 1.3%; caches
// that fit it are re-read from it, where the 3-tile ring measured 3-4% faster
// (prefill Q8K and Q2K at 32K).
constexpr uint64_t INFINITY_CACHE_BYTES = uint64_t(256) << 20;
static uint64_t kv_cache_bytes(const SparseMlaParams* p) {
  const uint64_t rows = (uint64_t)p->ORI_BLOCKS * p->PAGE + (uint64_t)p->CMP_BLOCKS * (p->PAGE / p->RATIO);
  return rows * (uint64_t)p->D * 2u;
}

static SparseArgs make_args(const SparseMlaParams* p, const void* q, const void* ori_kv,
                            const void* cmp_kv, const int32_t* idx, const int32_t* ot,
                            const int32_t* ct, const int32_t* cu, const int32_t* so,
                            const int32_t* sc, const int32_t* rs, const int32_t* otl,
                            const float* sinks, void* out) {
  SparseArgs a;
  a.q = q;
  a.ori_kv = ori_kv;
  a.cmp_kv = cmp_kv;
  a.indices = idx;
  a.ori_table = ot;
  a.cmp_table = ct;
  a.cu = cu;
  a.seq_ori = so;
  a.seq_cmp = sc;
  a.residual = rs;
  a.ori_topk_length = otl;
  a.sinks = sinks;
  a.out = out;
  a.lse = p->softmax_lse;
  a.debug_rows = p->debug_rows;
  a.B = p->B;
  a.T = p->T;
  a.H = p->H;
  a.D = p->D;
  a.PAGE = p->PAGE;
  a.RATIO = p->RATIO;
  a.table_width = p->MAX_SEQ / p->PAGE;
  a.ori_blocks = p->ORI_BLOCKS;
  a.cmp_blocks = p->CMP_BLOCKS;
  a.WINDOW = p->WINDOW;
  a.TOPK = p->TOPK;
  a.S = p->S;
  a.BM = p->BM;
  a.list_pad = (p->WINDOW + p->TOPK + 255) / 256 * 256;
  a.plan_rows = nullptr;
  a.plan_count = nullptr;
  a.partials = nullptr;
  const Split split = choose_split(p);
  a.parts = split.parts;
  a.split_from = (int32_t)split.split_from;
  a.ring = p->ring != 0 ? p->ring : (kv_cache_bytes(p) > INFINITY_CACHE_BYTES ? 4 : 3);
  // Non-temporal KV row loads (one-item kernel; and Q and O accesses in the
  // persistent kernel) when requests have at most 16 query tokens on average
  // (decode and multi-token decode: B64 x 6 62.7 -> 59.8 µs, 85 keys 72.4 ->
  // 69.3 µs, B128 x 6 on the persistent kernel 113.2 -> 104.4 µs). Many tokens
  // of one request share its rows through the L2, which these loads give up:
  // one request of 500 tokens measured 58.0 -> 63.4 µs with them (and the
  // persistent prefill kernel 43% slower).
  a.stream_kv = (int64_t)p->T <= 16 * (int64_t)p->B ? 1 : 0;
  a.scale = p->scale;
  return a;
}

// Plan workspace, each slice starting on a 256-byte boundary:
//   [T] counts | [T][list_pad] row lists | partial records of split keys,
//   [split keys][parts][BM / 16 output waves][BM * D / (BM / 16) + 2 * BM]
//   bytes: per (key, part) 2 * BM * D + BM * BM / 2 (each output wave's
//   normalised O slice in the storage dtype, and the running max and
//   denominator of every head, store_record).
static size_t round256(size_t n) { return (n + 255) / 256 * 256; }
static size_t plan_count_bytes(int64_t T) { return round256((size_t)T * 4); }
static size_t plan_rows_bytes(const SparseMlaParams* p) {
  const int64_t list_pad = (p->WINDOW + p->TOPK + 255) / 256 * 256;
  return (size_t)p->T * (size_t)list_pad * 4;
}
static size_t partial_bytes(const SparseMlaParams* p, const Split& split) {
  const int64_t tiles = (int64_t)p->T * (p->H / p->BM);
  if (split.parts < 2) return 0;
  return (size_t)(tiles - split.split_from) * (size_t)split.parts * (size_t)record_bytes_per_part(p);
}
static size_t plan_bytes(const SparseMlaParams* p) {
  return round256(plan_count_bytes(p->T) + plan_rows_bytes(p)) + partial_bytes(p, choose_split(p));
}

// LDS of one workgroup (the KV ring, P slots and the row list) must fit the
// 160 KiB a gfx950 CU holds.
constexpr size_t LDS_BYTES = 160 * 1024;
// The static LDS of each kernel is queried once per process (a function-local
// static per kernel, initialised thread-safely) instead of on every launch.
template <auto Kernel>
static int fits_lds(size_t dynamic_bytes) {
  static const std::pair<hipError_t, size_t> info = [] {
    hipFuncAttributes attr{};
    const hipError_t e = hipFuncGetAttributes(&attr, (const void*)Kernel);
    return std::make_pair(e, (size_t)attr.sharedSizeBytes);
  }();
  if (info.first != hipSuccess) return (int)info.first;
  return info.second + dynamic_bytes <= LDS_BYTES ? AFA_OK : AFA_E_SHAPE;
}

// Compute units of the current device (one persistent workgroup each).
static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  return cus;
}

// KV ring of the persistent kernel for these arguments: a.ring tiles (4 keeps
// two chunks in flight, for rows streamed from HBM) where the row-list ring of
// 5 lists fits next to them, else 3 (4 lists); 0 when neither fits.
template <int DT, int D, int NQ, int NP>
static int persistent_ring(const SparseArgs& a) {
  const size_t lds = (size_t)a.list_pad * sizeof(uint32_t);
  if (a.ring == 4 && fits_lds<sparse_mla_persistent_kernel<DT, D, NQ, NP, 4, false>>(5 * lds) == AFA_OK) return 4;
  return fits_lds<sparse_mla_persistent_kernel<DT, D, NQ, NP, 3, false>>(4 * lds) == AFA_OK ? 3 : 0;
}

// The persistent kernel over the plan at a.plan_count / a.plan_rows: one
// workgroup per CU (at most one per item).
template <int DT, int D, int NQ, int NP, bool CLAMP = false>
static int launch_persistent(const SparseArgs& a, int ring, hipStream_t stream) {
  const size_t lds = (size_t)a.list_pad * sizeof(uint32_t);
  static const int cus = device_cus();
  const int64_t items = (int64_t)a.T * (a.H / a.BM);
  const unsigned grid = (unsigned)std::min<int64_t>(cus, items);
  // Calls of few query tokens per request (a.stream_kv) take the form with
  // non-temporal KV, Q and O accesses at D = 512 (decode B128 x 6 113.2 ->
  // 104.4 µs); prefill keeps ordinary ones (non-temporal KV loads made it 43%
  // slower: consecutive tokens share rows through the L2).
  if constexpr (D == 512) {
    if (a.stream_kv) {
      if (ring == 4)
        hipLaunchKernelGGL((sparse_mla_persistent_kernel<DT, D, NQ, NP, 4, CLAMP, true>), dim3(grid),
                           dim3((NQ + NP) * 64), 5 * lds, stream, a);
      else
        hipLaunchKernelGGL((sparse_mla_persistent_kernel<DT, D, NQ, NP, 3, CLAMP, true>), dim3(grid),
                           dim3((NQ + NP) * 64), 4 * lds, stream, a);
      return (int)hipGetLastError();
    }
  }
  if (ring == 4)
    hipLaunchKernelGGL((sparse_mla_persistent_kernel<DT, D, NQ, NP, 4, CLAMP>), dim3(grid), dim3((NQ + NP) * 64), 5 * lds,
                       stream, a);
  else
    hipLaunchKernelGGL((sparse_mla_persistent_kernel<DT, D, NQ, NP, 3, CLAMP>), dim3(grid), dim3((NQ + NP) * 64), 4 * lds,
                       stream, a);
  return (int)hipGetLastError();
}

// After the one-item kernel: the merge of split keys, if any.
template <int DT, int D, int NQ, int NP>
static int after_one_item(const SparseArgs& a, int64_t tiles, hipStream_t stream) {
  if (a.parts < 2) return (int)hipGetLastError();
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL((sparse_merge_kernel<DT, D, NQ, NP>), dim3((unsigned)((tiles - a.split_from) * NP * NQ)),
                     dim3(merge_threads<D, NP>()), 0, stream, a);
  return (int)hipGetLastError();
}

template <int DT, int D, int NQ, int NP>
static int launch_fused(const SparseArgs& a, hipStream_t stream) {
  const size_t lds = (size_t)a.list_pad * sizeof(uint32_t);
  const int64_t tiles = (int64_t)a.T * (a.H / a.BM);
  if (a.plan_rows != nullptr && a.parts == 1) {
    // Plan kernel, then the persistent kernel over the plan when every CU gets
    // at least two items (the persistent form removes the per-item start,
    // which outweighs a second kernel only then) and a KV ring with its
    // row-list ring fits. Otherwise (and for split keys) the
    // one-item-per-workgroup kernel resolves its own rows.
    static const int cus = device_cus();
    const int ring = persistent_ring<DT, D, NQ, NP>(a);
    if (tiles >= 2 * (int64_t)cus && ring != 0) {
      constexpr int PLAN_THREADS = 64;
      hipLaunchKernelGGL((sparse_plan_kernel<PLAN_THREADS>), dim3((unsigned)a.T), dim3(PLAN_THREADS), lds, stream, a);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return (int)e;
      return launch_persistent<DT, D, NQ, NP>(a, ring, stream);
    }
  }
  // One workgroup per item (whole keys, then the parts of split keys): a
  // 4-tile ring (two chunks in flight) where it fits, since the kernel runs
  // short streams whose rows mostly come from HBM; then the merge of split keys.
  const int64_t items = a.split_from + (tiles - a.split_from) * a.parts;
  const unsigned blocks = (unsigned)items;
  // The non-temporal KV form (a.stream_kv) exists for D = 512, the decode
  // shape; a uniform branch in the fetch instead of a second kernel cost
  // 8-11% on every call of the first.
  if (fits_lds<sparse_mla_kernel<DT, D, NQ, NP, 4>>(lds) == AFA_OK) {
    if constexpr (D == 512) {
      if (a.stream_kv) {
        hipLaunchKernelGGL((sparse_mla_kernel<DT, D, NQ, NP, 4, true>), dim3(blocks), dim3((NQ + NP) * 64), lds, stream,
                           a);
        return after_one_item<DT, D, NQ, NP>(a, tiles, stream);
      }
    }
    hipLaunchKernelGGL((sparse_mla_kernel<DT, D, NQ, NP, 4>), dim3(blocks), dim3((NQ + NP) * 64), lds, stream, a);
  } else {
    const int fit = fits_lds<sparse_mla_kernel<DT, D, NQ, NP, 3>>(lds);
    if (fit) return fit;
    if constexpr (D == 512) {
      if (a.stream_kv) {
        hipLaunchKernelGGL((sparse_mla_kernel<DT, D, NQ, NP, 3, true>), dim3(blocks), dim3((NQ + NP) * 64), lds, stream,
                           a);
        return after_one_item<DT, D, NQ, NP>(a, tiles, stream);
      }
    }
    hipLaunchKernelGGL((sparse_mla_kernel<DT, D, NQ, NP, 3>), dim3(blocks), dim3((NQ + NP) * 64), lds, stream, a);
  }
  return after_one_item<DT, D, NQ, NP>(a, tiles, stream);
}


// BM = 16 * NQ heads per workgroup: 4 score + 4 output waves for BM = 64,
// 2 + 2 for BM = 32.
template <int DT>
static int dispatch_d(const SparseArgs& a, hipStream_t s) {
  const bool four = a.BM == 64;
  switch (a.D) {
    case 128: return four ? launch_fused<DT, 128, 4, 4>(a, s) : launch_fused<DT, 128, 2, 2>(a, s);
    case 256: return four ? launch_fused<DT, 256, 4, 4>(a, s) : launch_fused<DT, 256, 2, 2>(a, s);
    default: return four ? launch_fused<DT, 512, 4, 4>(a, s) : launch_fused<DT, 512, 2, 2>(a, s);
  }
}

extern "C" int launch_sparse_mla(void* stream, const void* q, const void* ori_kv,
                                 const void* cmp_kv, const int32_t* cmp_sparse_indices,
                                 const int32_t* ori_block_table, const int32_t* cmp_block_table,
                                 const int32_t* cu_seqlens_q, const int32_t* seqused_ori_kv,
                                 const int32_t* seqused_cmp_kv, const int32_t* cmp_residual_kv,
                                 const int32_t* ori_topk_length, const float* sinks,
                                 void* attention_out, void* workspace,
                                 const SparseMlaParams* params) {
  const int status = check_sparse(params);
  if (status) return status;
  if (!q || !ori_kv || !cmp_kv || !cmp_sparse_indices || !ori_block_table || !cmp_block_table ||
      !cu_seqlens_q || !seqused_ori_kv || !seqused_cmp_kv || !cmp_residual_kv ||
      !ori_topk_length || !sinks || !attention_out)
    return AFA_E_NULL;
  SparseArgs a = make_args(params, q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table,
                           cmp_block_table, cu_seqlens_q, seqused_ori_kv, seqused_cmp_kv,
                           cmp_residual_kv, ori_topk_length, sinks, attention_out);
  // With a workspace the row lists come from the plan kernel; the debug image
  // is written by the fused setup, so a debug call resolves rows in place.
  if (workspace != nullptr && params->debug_rows == nullptr) {
    char* w = (char*)workspace;
    a.plan_count = (int32_t*)w;
    a.plan_rows = (uint32_t*)(w + plan_count_bytes(params->T));
    if (a.parts > 1) a.partials = w + round256(plan_count_bytes(params->T) + plan_rows_bytes(params));
  } else {
    a.parts = 1;
    a.split_from = a.T * (a.H / a.BM);
  }
  hipStream_t s = (hipStream_t)stream;
  return params->dtype == AFA_DTYPE_BF16 ? dispatch_d<DT_BF16>(a, s) : dispatch_d<DT_F16>(a, s);
}

// Scratch of the allocation-free entry point: the workspace of one call (the
// row-list plan and any split records) in a file-scope device array, so the
// call needs no allocation. Each GPU holds its own copy until the process ends;
// every call on a GPU reuses it, so calls that overlap on one GPU race. Nothing
// in it has to start at zero: each call writes every count, list entry and
// record it later reads.
constexpr size_t SCRATCH_BYTES = size_t(32) << 20;
static_assert(SCRATCH_BYTES == AFA_SCRATCH_BYTES, "the header states the scratch size");
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

// Device address of the current GPU's copy of `scratch`, resolved once per
// device with hipGetSymbolAddress (the array's name is a host-side stand-in,
// not a device address, and must never be passed to a kernel or a copy).
static int scratch_address(void** out) {
  constexpr int MAX_DEVICES = 64;
  static std::atomic<void*> address[MAX_DEVICES];
  static std::mutex resolve;
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return (int)e;
  if (device < 0 || device >= MAX_DEVICES) return AFA_E_SHAPE;
  void* p = address[device].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> guard(resolve);
    p = address[device].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (p == nullptr) return (int)hipErrorInvalidSymbol;
      address[device].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return AFA_OK;
}

extern "C" int launch_sparse_mla_noalloc(void* stream, const void* q, const void* ori_kv,
                                         const void* cmp_kv, const int32_t* cmp_sparse_indices,
                                         const int32_t* ori_block_table, const int32_t* cmp_block_table,
                                         const int32_t* cu_seqlens_q, const int32_t* seqused_ori_kv,
                                         const int32_t* seqused_cmp_kv, const int32_t* cmp_residual_kv,
                                         const int32_t* ori_topk_length, const float* sinks,
                                         void* attention_out, const SparseMlaParams* params) {
  const int status = check_sparse(params);
  if (status) return status;
  if (plan_bytes(params) > SCRATCH_BYTES) return AFA_E_WORKSPACE;
  void* workspace = nullptr;
  const int resolved = scratch_address(&workspace);
  if (resolved) return resolved;
  return launch_sparse_mla(stream, q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table, cmp_block_table,
                           cu_seqlens_q, seqused_ori_kv, seqused_cmp_kv, cmp_residual_kv, ori_topk_length, sinks,
                           attention_out, workspace, params);
}

extern "C" int launch_sparse_mla_gather(void* stream, const void* ori_kv, const void* cmp_kv,
                                        const int32_t* cmp_sparse_indices,
                                        const int32_t* ori_block_table,
                                        const int32_t* cmp_block_table,
                                        const int32_t* cu_seqlens_q,
                                        const int32_t* seqused_ori_kv,
                                        const int32_t* seqused_cmp_kv,
                                        const int32_t* cmp_residual_kv,
                                        const int32_t* ori_topk_length, void* kv_out,
                                        float* bias_out, const SparseMlaParams* params) {
  const int status = check_sparse(params);
  if (status) return status;
  if (!ori_kv || !cmp_kv || !cmp_sparse_indices || !ori_block_table || !cmp_block_table ||
      !cu_seqlens_q || !seqused_ori_kv || !seqused_cmp_kv || !cmp_residual_kv ||
      !ori_topk_length || !kv_out || !bias_out)
    return AFA_E_NULL;
  SparseArgs a = make_args(params, nullptr, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table,
                           cmp_block_table, cu_seqlens_q, seqused_ori_kv, seqused_cmp_kv,
                           cmp_residual_kv, ori_topk_length, nullptr, nullptr);
  a.debug_rows = nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (params->dtype == AFA_DTYPE_BF16)
    hipLaunchKernelGGL(sparse_gather_kernel<DT_BF16>, dim3(params->T), dim3(256), 0, s, a, kv_out,
                       bias_out);
  else
    hipLaunchKernelGGL(sparse_gather_kernel<DT_F16>, dim3(params->T), dim3(256), 0, s, a, kv_out,
                       bias_out);
  return (int)hipGetLastError();
}

// Plan only: the row-list plan of launch_sparse_mla's workspace (layout in
// include/ascendflow_amd.h), written by the same plan kernel.
extern "C" int launch_sparse_mla_plan(void* stream, const int32_t* cmp_sparse_indices,
                                      const int32_t* ori_block_table, const int32_t* cmp_block_table,
                                      const int32_t* cu_seqlens_q, const int32_t* seqused_ori_kv,
                                      const int32_t* seqused_cmp_kv, const int32_t* cmp_residual_kv,
                                      const int32_t* ori_topk_length, void* workspace,
                                      const SparseMlaParams* params) {
  const int status = check_sparse(params);
  if (status) return status;
  if (!cmp_sparse_indices || !ori_block_table || !cmp_block_table || !cu_seqlens_q || !seqused_ori_kv ||
      !seqused_cmp_kv || !cmp_residual_kv || !ori_topk_length || !workspace)
    return AFA_E_NULL;
  SparseArgs a = make_args(params, nullptr, nullptr, nullptr, cmp_sparse_indices, ori_block_table, cmp_block_table,
                           cu_seqlens_q, seqused_ori_kv, seqused_cmp_kv, cmp_residual_kv, ori_topk_length, nullptr,
                           nullptr);
  a.plan_count = (int32_t*)workspace;
  a.plan_rows = (uint32_t*)((char*)workspace + plan_count_bytes(params->T));
  constexpr int PLAN_THREADS = 64;
  hipLaunchKernelGGL((sparse_plan_kernel<PLAN_THREADS>), dim3((unsigned)a.T), dim3(PLAN_THREADS),
                     (size_t)a.list_pad * sizeof(uint32_t), (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

template <int DT>
static int dispatch_planned(const SparseArgs& a, hipStream_t s) {
  auto run = [&](auto launch_ring, auto launch) {
    const int ring = launch_ring(a);
    return ring == 0 ? (int)AFA_E_SHAPE : launch(a, ring, s);
  };
  const bool four = a.BM == 64;
  switch (a.D) {
    case 128:
      return four ? run(persistent_ring<DT, 128, 4, 4>, launch_persistent<DT, 128, 4, 4, true>)
                  : run(persistent_ring<DT, 128, 2, 2>, launch_persistent<DT, 128, 2, 2, true>);
    case 256:
      return four ? run(persistent_ring<DT, 256, 4, 4>, launch_persistent<DT, 256, 4, 4, true>)
                  : run(persistent_ring<DT, 256, 2, 2>, launch_persistent<DT, 256, 2, 2, true>);
    default:
      return four ? run(persistent_ring<DT, 512, 4, 4>, launch_persistent<DT, 512, 4, 4, true>)
                  : run(persistent_ring<DT, 512, 2, 2>, launch_persistent<DT, 512, 2, 2, true>);
  }
}

extern "C" int launch_sparse_mla_planned(void* stream, const void* q, const void* ori_kv, const void* cmp_kv,
                                         const float* sinks, void* attention_out, const void* workspace,
                                         const SparseMlaParams* params) {
  const int status = check_sparse(params);
  if (status) return status;
  if (params->debug_rows != nullptr) return AFA_E_SHAPE;  // the plan path writes no debug image
  if (!q || !ori_kv || !cmp_kv || !sinks || !attention_out || !workspace) return AFA_E_NULL;
  SparseArgs a = make_args(params, q, ori_kv, cmp_kv, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                           nullptr, sinks, attention_out);
  a.plan_count = (int32_t*)workspace;
  a.plan_rows = (uint32_t*)((char*)workspace + plan_count_bytes(params->T));
  a.parts = 1;
  a.split_from = a.T * (a.H / a.BM);
  hipStream_t s = (hipStream_t)stream;
  return params->dtype == AFA_DTYPE_BF16 ? dispatch_planned<DT_BF16>(a, s) : dispatch_planned<DT_F16>(a, s);
}

extern "C" int launch_gather_probe(void* stream, const void* ori_kv, const void* cmp_kv, const void* workspace,
                                   const SparseMlaParams* params, int32_t grid, int32_t depth, int32_t balanced,
                                   uint32_t* sums) {
  const int status = check_sparse(params);
  if (status) return status;
  if (!ori_kv || !cmp_kv || !workspace || !sums) return AFA_E_NULL;
  if (params->D != 512 || params->BM != params->H) return AFA_E_SHAPE;  // 1 KiB rows, one item per token
  if (grid < 1 || (int64_t)grid * PROBE_ITEMS < params->T + (balanced ? grid : 0)) return AFA_E_SHAPE;
  const int list_pad = (params->WINDOW + params->TOPK + 255) / 256 * 256;
  const int32_t* counts = (const int32_t*)workspace;
  const uint32_t* lists = (const uint32_t*)((const char*)workspace + plan_count_bytes(params->T));
  const size_t lds = (size_t)PROBE_ITEMS * list_pad * sizeof(uint32_t);
  hipStream_t s = (hipStream_t)stream;
  const char* o = (const char*)ori_kv;
  const char* c = (const char*)cmp_kv;
#define AFA_PROBE(D)                                                                                          \
  case D:                                                                                                     \
    if (fits_lds<gather_probe_kernel<D>>(lds) != AFA_OK) return AFA_E_SHAPE;                                 \
    hipLaunchKernelGGL(gather_probe_kernel<D>, dim3((unsigned)grid), dim3(256), lds, s, o, c, counts, lists,    \
                       list_pad, params->T, balanced, sums);                                                  \
    break;
  switch (depth) {
    AFA_PROBE(1) AFA_PROBE(2) AFA_PROBE(4) AFA_PROBE(6) AFA_PROBE(8)
    default: return AFA_E_SHAPE;
  }
#undef AFA_PROBE
  return (int)hipGetLastError();
}

extern "C" int kernel_config_sparse_mla(int64_t cfg[5]) {
  if (!cfg) return AFA_E_NULL;
  cfg[0] = 13;  // external tensors
  cfg[1] = 0;   // runtime size parameters: all sizes travel in SparseMlaParams
  cfg[2] = 1;   // optional workspace: the per-token row-list plan
  cfg[3] = 256; // MI355X compute units
  cfg[4] = 4;   // SIMDs per compute unit
  return AFA_OK;
}

extern "C" int workspace_size_sparse_mla(uint64_t* bytes, const SparseMlaParams* params) {
  if (!bytes) return -1;
  const int status = check_sparse(params);
  if (status) return status;
  *bytes = plan_bytes(params);
  return AFA_OK;
}

// Launch-ABI description in the reference's metadata schema
// (src/backend/abi.py:19-59): tensors with dtype, shape (named axes, bound
// consistently across tensors by the caller), layout and access; runtime
// size parameters with minimum and multiple (none here: the reference
// specialises every sparse size at compile time, and this library takes them
// in SparseMlaParams, listed under "params_struct"); "DTYPE" is one of
// "dtypes". CMP_PAGE = PAGE / RATIO, TABLE_WIDTH = MAX_SEQ / PAGE, B1 = B + 1.
extern "C" const char* kernel_metadata_sparse_mla(void) {
  return "{\"version\":1,\"name\":\"sparse_mla\",\"target\":\"gfx950\",\"kind\":\"mixed\","
         "\"groups\":256,\"disjoint_external\":true,\"device_resources\":null,"
         "\"dtypes\":{\"DTYPE\":[\"bf16\",\"f16\"]},\"tensors\":["
         "{\"name\":\"q\",\"dtype\":\"DTYPE\",\"shape\":[\"T\",\"H\",\"D\"],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"ori_kv\",\"dtype\":\"DTYPE\",\"shape\":[\"ORI_BLOCKS\",\"PAGE\",1,\"D\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"cmp_kv\",\"dtype\":\"DTYPE\",\"shape\":[\"CMP_BLOCKS\",\"CMP_PAGE\",1,\"D\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"cmp_sparse_indices\",\"dtype\":\"i32\",\"shape\":[\"T\",1,\"TOPK\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"ori_block_table\",\"dtype\":\"i32\",\"shape\":[\"B\",\"TABLE_WIDTH\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"cmp_block_table\",\"dtype\":\"i32\",\"shape\":[\"B\",\"TABLE_WIDTH\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"cu_seqlens_q\",\"dtype\":\"i32\",\"shape\":[\"B1\"],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"seqused_ori_kv\",\"dtype\":\"i32\",\"shape\":[\"B\"],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"seqused_cmp_kv\",\"dtype\":\"i32\",\"shape\":[\"B\"],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"cmp_residual_kv\",\"dtype\":\"i32\",\"shape\":[\"B\"],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"ori_topk_length\",\"dtype\":\"i32\",\"shape\":[\"T\",1],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"sinks\",\"dtype\":\"f32\",\"shape\":[\"H\"],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"attention_out\",\"dtype\":\"DTYPE\",\"shape\":[\"T\",\"H\",\"D\"],"
         "\"layout\":\"linear\",\"access\":\"write\"}],"
         "\"parameters\":[],"
         "\"params_struct\":{\"name\":\"SparseMlaParams\",\"fields\":[\"B\",\"T\",\"H\",\"D\","
         "\"PAGE\",\"RATIO\",\"MAX_SEQ\",\"ORI_BLOCKS\",\"CMP_BLOCKS\",\"WINDOW\",\"TOPK\",\"S\","
         "\"BM\",\"dtype\",\"scale\",\"parts\",\"ring\",\"debug_rows\",\"softmax_lse\"]},"
         "\"workspace\":true}";
}
