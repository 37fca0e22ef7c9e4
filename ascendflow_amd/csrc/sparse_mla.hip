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
//      row list of physical row ids;
//   2. stream the listed rows through a double-buffered, XOR-swizzled LDS
//      tile of CHUNK rows with 16-byte coalesced loads (one wave reads whole
//      1 KiB rows when D = 512);
//   3. each wave owns 16 heads: S^T[rows, heads] = KV * Q^T on
//      v_mfma_f32_16x16x32_{bf16,f16} with Q resident in registers;
//   4. FP32 online softmax per head in registers (exp2 domain), the sink
//      seeding the running max and contributing e^(sink-m) once;
//   5. P (rounded to the storage dtype, round-to-nearest-even) feeds
//      O^T[d, heads] += V^T * P^T directly from the S^T accumulators; V^T
//      fragments come from the same LDS rows through ds_read_b64_tr_b16;
//   6. O = O_acc * (1 / l), rounded to the storage dtype.
//
// K and V are the same gathered rows; each row is read from global memory
// once per workgroup and from LDS twice (once per contraction).
#include <type_traits>

#include "common.h"
#include "../../include/ascendflow_amd.h"

namespace afa {

constexpr int CHUNK = 32;                 // rows per LDS stage
constexpr uint32_t CMP_BIT = 0x80000000u; // row-list tag: row lives in cmp_kv
constexpr float LOG2E = 1.4426950408889634f;

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
  int32_t* debug_rows;
  int32_t B, T, H, D, PAGE, RATIO, table_width, ori_blocks, cmp_blocks, WINDOW, TOPK, S, BM;
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

// The same request for a whole workgroup with one round of parallel loads:
// since cu is non-decreasing and cu[0] = 0 <= token, the answer is
// #{b in [0, B): cu[b] <= token} - 1.
template <int NW>
__device__ __forceinline__ int request_by_count(const SparseArgs& a, int token, int* scratch) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int n = 0;
  for (int b = tid; b < a.B; b += NW * 64) n += a.cu[b] <= token ? 1 : 0;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) n += __shfl_xor(n, d);
  if (lane == 0) scratch[wave] = n;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) total += scratch[w];
  return total - 1;
}

// query_metadata (gather.py:8-35) and the compressed bound (attention.py:339-341)
// of a token whose request is `batch`.
__device__ __forceinline__ Geometry token_geometry(const SparseArgs& a, int token, int batch) {
  const int lo = batch;
  Geometry g;
  g.batch = lo;
  const int begin = a.cu[lo], count = a.cu[lo + 1] - begin, offset = token - begin;
  g.right = max(0, a.seq_ori[lo] - count + offset + 1);
  int visible = min(a.WINDOW, g.right);
  const int narrowed = a.ori_topk_length[token];
  if (narrowed > 0) visible = min(visible, narrowed);
  g.visible = visible;
  const int available = a.seq_cmp[lo];
  const int end = available * a.RATIO + a.residual[lo];
  g.cutoff = max(0, end - count + offset + 1) / a.RATIO;
  g.count_cmp = max(0, min(a.TOPK, min(available, g.cutoff)));
  return g;
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

// Lazy rescaling threshold (log2 units): the running max used for exp2 is only
// raised, and O/l rescaled, once some head's max exceeds it by more than
// TAU, so P stays <= 2^TAU; the final O/l is independent of the reference point.
constexpr float TAU = 8.0f;

// s_waitcnt immediate for lgkmcnt(0) alone (gfx9 encoding: vmcnt[3:0] |
// expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14, all other fields at max).
constexpr int WAIT_LGKM0 = 0xC07F;
// Workgroup barrier without the memory fence of __syncthreads(): global loads
// of later chunks stay in flight across it. The caller's own LDS stores are
// complete (lgkmcnt(0)) before it signals; the empty asm statements keep the
// compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

constexpr int NSTAGE = 3;  // KV chunk buffers in LDS
constexpr int LOOK = 12;    // V^T fragment-read lookahead (d-tiles) in the PV loop
constexpr int LOOK_QK = 4;  // KV fragment-read lookahead (k-steps) in the QK loop

// Workgroup = one (token, BM-head tile). HG head groups of HT*16 heads and DS
// feature parts: wave w owns heads [16*HT*(w % HG), +16*HT) and features
// [(w / HG) * D/DS, +D/DS). Each KV fragment read from LDS feeds HT MFMAs (one
// per 16-head tile). With DS > 1 the DS waves of a head group add their
// partial scores through LDS, so each wave keeps only its share of Q and O.
//
// Software pipeline, one barrier per chunk c:
//   stash KV(c+1) -> barrier -> fetch KV(c+2) -> exchange partial S(c) ->
//   softmax(c) -> { QK(c+1) interleaved with PV(c) } -> publish partial S(c+1)
// so the LDS reads and MFMAs of two chunks overlap. KV uses a ring of NSTAGE
// buffers: when a wave stashes chunk c+1, the slowest wave is at worst still
// reading chunks c-1 (PV) and c (QK), which live in the other two buffers.
template <int DT, int D, int HG, int HT, int DS>
__global__ __launch_bounds__(HG * DS * 64) void sparse_mla_kernel(SparseArgs a) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x8 x8;
  typedef typename B16<DT>::x4 x4;
  constexpr int NW = HG * DS;
  constexpr int NT = NW * 64;
  constexpr int DP = D / DS;                   // features per wave
  constexpr int UNITS = D / 8;                 // 16-byte units per row
  constexpr int PIECES = CHUNK * UNITS / NT;   // 16-byte loads per thread per chunk
  constexpr int ROW_BYTES = D * 2;
  constexpr int QK_STEPS = DP / 32, PV_STEPS = DP / 16;
  static_assert(CHUNK * UNITS % NT == 0, "chunk must split evenly over the block");
  static_assert(UNITS >= 16, "swizzle needs at least 16 units per row");
  static_assert(DP % 32 == 0 && DP / 8 % 16 == 0, "feature part must hold whole swizzle groups");

  __shared__ __attribute__((aligned(16))) uint8_t kv_lds[NSTAGE][CHUNK * ROW_BYTES];
  __shared__ __attribute__((aligned(16))) f32x4 s_xchg[DS > 1 ? 2 : 1][DS > 1 ? NW : 1][DS > 1 ? 2 * HT : 1][64];
  __shared__ int wave_count[NW];
  extern __shared__ uint32_t row_list[];  // round_up(WINDOW + TOPK, CHUNK) entries

  const int tid = threadIdx.x;
  // The wave index is uniform; readfirstlane lets the compiler see that, so
  // branches on the wave's role are scalar branches.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 4, i16 = lane & 15;
  const int hg = wave % HG, part = wave / HG;
  const int head_tiles = a.H / a.BM;
  const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
  const int token = (int)(logical / head_tiles);
  const int head0 = (int)(logical % head_tiles) * a.BM;

  // ---- 1. Q fragments (B operand of S^T = KV * Q^T) for this wave's features,
  // issued first so their latency overlaps the request search and row list
  const int dbase = part * DP;
  const int hbase = head0 + hg * 16 * HT + i16;  // head of head tile ht: hbase + 16*ht
  x8 qf[HT][QK_STEPS];
  f32x4 o[HT][PV_STEPS];
  float m_run[HT], l_run[HT];
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    const scalar* q_row = (const scalar*)a.q + ((size_t)token * a.H + hbase + 16 * ht) * D + dbase + 8 * g;
#pragma unroll
    for (int j = 0; j < QK_STEPS; ++j) qf[ht][j] = *(const x8*)(q_row + 32 * j);
#pragma unroll
    for (int t = 0; t < PV_STEPS; ++t) o[ht][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[ht] = a.sinks[hbase + 16 * ht] * LOG2E;  // sink seeds the running max
    l_run[ht] = g == 0 ? 1.0f : 0.0f;              // e^(sink - m) counted once per head
  }
  const float scale_log2 = a.scale * LOG2E;

  __shared__ int request_scratch[NW];
  const Geometry geo = token_geometry(a, token, request_by_count<NW>(a, token, request_scratch));

  // ---- 2. compact the selected rows into the LDS row list -------------------
  const int slots = a.WINDOW + geo.count_cmp;
  int n_rows = 0;
  for (int s0 = 0; s0 < slots; s0 += NT) {
    const int s = s0 + tid;
    uint32_t entry = 0;
    const bool valid = s < slots && resolve_slot(a, geo, token, s, entry);
    const uint64_t mask = __ballot(valid);
    if (lane == 0) wave_count[wave] = __popcll(mask);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int c = wave_count[w];
      before += w < wave ? c : 0;
      total += c;
    }
    if (valid) {
      const int within = __popcll(mask & ((1ull << lane) - 1ull));
      row_list[n_rows + before + within] = entry;
    }
    n_rows += total;
    __syncthreads();
  }
  // Pad the last chunk with a real row so every load is unconditional; the
  // padded rows get -inf scores (P = 0) below.
  const int chunks = (n_rows + CHUNK - 1) / CHUNK;
  if (tid < chunks * CHUNK - n_rows) row_list[n_rows + tid] = row_list[0];
  if (a.debug_rows != nullptr && head0 == 0) {
    for (int s = tid; s < a.S; s += NT) {
      uint32_t entry = 0;
      const bool valid = s < slots && resolve_slot(a, geo, token, s, entry);
      int2 v = make_int2(-1, -1);
      if (valid) v = make_int2((entry & CMP_BIT) ? 1 : 0, (int)(entry & ~CMP_BIT));
      ((int2*)a.debug_rows)[(size_t)token * a.S + s] = v;
    }
  }
  __syncthreads();

  // ---- 3. KV movement: global -> registers -> swizzled LDS rows --------------
  // Each wave moves PIECES rows of a chunk. With D = 512 one wave load covers
  // exactly one 1 KiB row, so a wave takes PIECES consecutive rows whose list
  // entries and addresses are wave-uniform (scalar registers); the lanes only
  // add their 16-byte unit offset. Smaller D spreads one load over several rows.
  constexpr bool ROW_LOADS = (UNITS == 64);
  u32x4 pf[PIECES];
  const char* ori = (const char*)a.ori_kv;
  const char* cmp = (const char*)a.cmp_kv;
  const uint32_t kv_base = lds_address(kv_lds[0]);
  auto tile_address = [&](int chunk) {
    return opaque_uniform(kv_base + (uint32_t)(chunk % NSTAGE) * (CHUNK * ROW_BYTES));
  };
  // This lane's LDS offset inside a tile for piece p.
  uint32_t stash_offset[PIECES];
#pragma unroll
  for (int p = 0; p < PIECES; ++p) {
    const int flat = ROW_LOADS ? (wave * PIECES + p) * UNITS + lane : tid + p * NT;
    const int r = flat / UNITS, u = flat % UNITS;
    stash_offset[p] = (uint32_t)(r * ROW_BYTES + (swz(r, u) << 4));
  }
  auto fetch = [&](int chunk) {
    if constexpr (ROW_LOADS) {
      const int first = chunk * CHUNK + wave * PIECES;
#pragma unroll
      for (int p = 0; p < PIECES; ++p) {
        const uint32_t e = __builtin_amdgcn_readfirstlane(row_list[first + p]);
        const char* row = ((e & CMP_BIT) ? cmp : ori) + (size_t)(e & ~CMP_BIT) * ROW_BYTES;
        pf[p] = *(const u32x4*)(row + lane * 16);
      }
    } else {
#pragma unroll
      for (int p = 0; p < PIECES; ++p) {
        const int flat = tid + p * NT;
        const int r = flat / UNITS, u = flat % UNITS;
        const uint32_t e = row_list[chunk * CHUNK + r];
        const char* base = (e & CMP_BIT) ? cmp : ori;
        pf[p] = *(const u32x4*)(base + (size_t)(e & ~CMP_BIT) * ROW_BYTES + u * 16);
      }
    }
  };
  auto stash = [&](int chunk) {
    const uint32_t tile = tile_address(chunk);
#pragma unroll
    for (int p = 0; p < PIECES; ++p) *(AFA_LDS u32x4*)lds_at<u32x4>(opaque(tile + stash_offset[p])) = pf[p];
  };

  // LDS byte offsets inside a chunk tile. The swizzle only permutes units
  // within aligned groups of 16 (256 bytes), so every fragment address is a
  // per-lane base (depending on j & 3 or t & 7) plus a compile-time offset.
  const int ra = sigma(i16);                   // QK fragment row inside a 16-row tile
  const int rt = sigma(4 * g + (i16 >> 2));    // transposing-read row inside a tile
  const int ubase = dbase / 8;                 // first 16-byte unit of this wave's features
  uint32_t qk_base[4], tr_base[8];
#pragma unroll
  for (int b = 0; b < 4; ++b)
    qk_base[b] = (uint32_t)(ra * ROW_BYTES + ubase * 16 + (((4 * b + g) ^ (ra & 15)) << 4));
#pragma unroll
  for (int b = 0; b < 8; ++b)
    tr_base[b] = (uint32_t)(rt * ROW_BYTES + ubase * 16 + (((2 * b + ((i16 & 3) >> 1)) ^ (rt & 15)) << 4) + (i16 & 1) * 8);

  f32x4 s[2][HT];  // partial S^T [row tile][head tile] of the chunk QK last ran on
  auto qk_zero = [&]() {
#pragma unroll
    for (int rtile = 0; rtile < 2; ++rtile)
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) s[rtile][ht] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto publish = [&](int chunk) {
    if constexpr (DS > 1) {
#pragma unroll
      for (int rtile = 0; rtile < 2; ++rtile)
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) s_xchg[chunk & 1][wave][rtile * HT + ht][lane] = s[rtile][ht];
    }
  };
  // Full scores of the head group: the wave's own partial is still in s (QK of
  // the next chunk has not run yet) and the other part's is read back. IEEE
  // addition is commutative, so both waves of a head group hold bit-identical
  // sums and take identical softmax decisions.
  static_assert(DS <= 2, "score exchange assumes at most two feature parts");
  auto gather_scores = [&](int chunk, f32x4 (&out)[2][HT]) {
#pragma unroll
    for (int rtile = 0; rtile < 2; ++rtile)
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) {
        if constexpr (DS == 2)
          out[rtile][ht] = s[rtile][ht] + s_xchg[chunk & 1][hg + (1 - part) * HG][rtile * HT + ht][lane];
        else
          out[rtile][ht] = s[rtile][ht];
      }
  };

  // QK of one chunk into s, fragment reads LOOK_QK k-steps ahead of the MFMAs.
  auto qk_chunk = [&](uint32_t tile) {
    x8 ka0[QK_STEPS], ka1[QK_STEPS];
    uint32_t base[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) base[b] = opaque(tile + qk_base[b]);
    auto load = [&](int j) {
      const AFA_LDS uint8_t* q = lds_at<uint8_t>(base[j & 3]) + (j >> 2) * 256;
      ka0[j] = *(const AFA_LDS x8*)q;
      ka1[j] = *(const AFA_LDS x8*)(q + 16 * ROW_BYTES);
    };
    qk_zero();
#pragma unroll
    for (int j = 0; j < LOOK_QK && j < QK_STEPS; ++j) load(j);
#pragma unroll
    for (int j = 0; j < QK_STEPS; ++j) {
      if (j + LOOK_QK < QK_STEPS) load(j + LOOK_QK);
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) {
        s[0][ht] = B16<DT>::mfma(ka0[j], qf[ht][j], s[0][ht]);
        s[1][ht] = B16<DT>::mfma(ka1[j], qf[ht][j], s[1][ht]);
      }
    }
  };

  // One pipeline iteration for chunk c; MORE says whether chunk c + 1 exists.
  auto iteration = [&](int c, auto more_tag) {
    constexpr bool MORE = decltype(more_tag)::value;
    if constexpr (MORE) stash(c + 1);
    block_barrier();
    f32x4 sc[2][HT];
    gather_scores(c, sc);

    // First V^T fragments of PV(c); they depend on neither QK(c+1) nor softmax(c).
    uint32_t vbase[8];
    x4 vlo[PV_STEPS], vhi[PV_STEPS];
    auto load_step = [&](int t) {
      const AFA_LDS uint8_t* p = lds_at<uint8_t>(vbase[t & 7]) + (t >> 3) * 256;
      vlo[t] = B16<DT>::read_tr((const AFA_LDS void*)p);
      vhi[t] = B16<DT>::read_tr((const AFA_LDS void*)(p + 16 * ROW_BYTES));
    };
    auto v_first = [&]() {
      const uint32_t tile = tile_address(c);
#pragma unroll
      for (int b = 0; b < 8; ++b) vbase[b] = opaque(tile + tr_base[b]);
#pragma unroll
      for (int t = 0; t < LOOK && t < PV_STEPS; ++t) load_step(t);
    };

    // Online softmax of chunk c per head tile; this lane holds the chunk rows
    // sigma(4g+i) and 16 + sigma(4g+i) of head hbase + 16*ht. The running max
    // (log2 units) starts at the sink and is raised (with O and l rescaled)
    // only when a head's max exceeds it by more than TAU. Since the scale is
    // positive, the chunk max is taken on the raw scores and the scale is
    // applied inside the exponent's FMA. Only the last chunk holds padding.
    x8 pf8[HT];
    auto softmax = [&]() {
      const int live = n_rows - c * CHUNK;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) {
        float x0[4], x1[4];
        float cmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x0[i] = sc[0][ht][i];
          x1[i] = sc[1][ht][i];
          if constexpr (!MORE) {
            const int row = sigma(4 * g + i);
            x0[i] = (row < live) ? x0[i] : -INFINITY;
            x1[i] = (16 + row < live) ? x1[i] : -INFINITY;
          }
          cmax = fmaxf(cmax, fmaxf(x0[i], x1[i]));
        }
        cmax = max_over_lane_groups(cmax);
        const float m_new = fmaxf(m_run[ht], cmax * scale_log2);
        if (__ballot(m_new > m_run[ht] + TAU) != 0ull) {
          const float alpha = fast_exp2(m_run[ht] - m_new);
          l_run[ht] *= alpha;
#pragma unroll
          for (int t = 0; t < PV_STEPS; ++t) o[ht][t] *= alpha;
          m_run[ht] = m_new;
        }
        const float neg_m = -m_run[ht];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p0 = fast_exp2(__builtin_fmaf(x0[i], scale_log2, neg_m));
          const float p1 = fast_exp2(__builtin_fmaf(x1[i], scale_log2, neg_m));
          psum += p0 + p1;
          pf8[ht][i] = (scalar)p0;
          pf8[ht][4 + i] = (scalar)p1;
        }
        l_run[ht] += psum;
      }
    };

    // QK(c+1) is issued first so its MFMAs run under the softmax of chunk c;
    // the gather of chunk c+2 and the first V^T fragments of PV(c) go out
    // before the softmax, which depends on neither.
    if constexpr (MORE) qk_chunk(tile_address(c + 1));
    if (c + 2 < chunks) fetch(c + 2);
    v_first();
    softmax();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MORE) publish(c + 1);

    // PV(c): V^T fragment reads LOOK steps ahead of their MFMAs; scheduling
    // barriers pin that distance so the registers in flight stay bounded.
#pragma unroll
    for (int t = 0; t < PV_STEPS; ++t) {
      if (t + LOOK < PV_STEPS) load_step(t + LOOK);
      const x8 v = {vlo[t][0], vlo[t][1], vlo[t][2], vlo[t][3], vhi[t][0], vhi[t][1], vhi[t][2], vhi[t][3]};
#pragma unroll
      for (int ht = 0; ht < HT; ++ht) o[ht][t] = B16<DT>::mfma(v, pf8[ht], o[ht][t]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- 4. pipelined chunk loop ----------------------------------------------
  if (chunks > 0) {
    fetch(0);
    stash(0);
    if (chunks > 1) fetch(1);
    block_barrier();
    qk_chunk(tile_address(0));
    publish(0);
    for (int c = 0; c + 1 < chunks; ++c) iteration(c, std::true_type{});
    iteration(chunks - 1, std::false_type{});
  }

  // ---- 5. normalise and store: this lane holds d = dbase + 16t + 4g + i.
#pragma unroll
  for (int ht = 0; ht < HT; ++ht) {
    const float inv = 1.0f / sum_over_lane_groups(l_run[ht]);
    scalar* out_row = (scalar*)a.out + ((size_t)token * a.H + hbase + 16 * ht) * D + dbase + 4 * g;
#pragma unroll
    for (int t = 0; t < PV_STEPS; ++t) {
      x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (scalar)(o[ht][t][i] * inv);
      *(x4*)(out_row + 16 * t) = v;
    }
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
  if (p->S < p->WINDOW + p->TOPK) return AFA_E_SHAPE;
  if (p->ORI_BLOCKS <= 0 || p->CMP_BLOCKS <= 0) return AFA_E_SHAPE;
  if ((int64_t)p->ORI_BLOCKS * p->PAGE >= (int64_t)CMP_BIT) return AFA_E_SHAPE;
  if ((int64_t)p->CMP_BLOCKS * (p->PAGE / p->RATIO) >= (int64_t)CMP_BIT) return AFA_E_SHAPE;
  if (!(p->scale > 0.0f)) return AFA_E_SHAPE;
  if ((int64_t)p->T * (p->H / p->BM) > 0x7fffffffLL) return AFA_E_SHAPE;
  return AFA_OK;
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
  a.scale = p->scale;
  return a;
}

template <int DT, int D, int HG, int HT, int DS>
static int launch_fused(const SparseArgs& a, hipStream_t stream) {
  const int list = (a.WINDOW + a.TOPK + CHUNK - 1) / CHUNK * CHUNK;
  const size_t lds = (size_t)list * sizeof(uint32_t);
  const unsigned blocks = (unsigned)a.T * (unsigned)(a.H / a.BM);
  hipLaunchKernelGGL((sparse_mla_kernel<DT, D, HG, HT, DS>), dim3(blocks), dim3(HG * DS * 64),
                     lds, stream, a);
  return (int)hipGetLastError();
}

// BM = 16 * HG * HT heads per workgroup.
template <int DT>
static int dispatch_d(const SparseArgs& a, hipStream_t s) {
  const bool four = a.BM == 64;
  switch (a.D) {
    case 128: return four ? launch_fused<DT, 128, 2, 2, 1>(a, s) : launch_fused<DT, 128, 1, 2, 1>(a, s);
    case 256: return four ? launch_fused<DT, 256, 2, 2, 2>(a, s) : launch_fused<DT, 256, 1, 2, 2>(a, s);
    default: return four ? launch_fused<DT, 512, 4, 1, 2>(a, s) : launch_fused<DT, 512, 2, 1, 2>(a, s);
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
  (void)workspace;
  const int status = check_sparse(params);
  if (status) return status;
  if (!q || !ori_kv || !cmp_kv || !cmp_sparse_indices || !ori_block_table || !cmp_block_table ||
      !cu_seqlens_q || !seqused_ori_kv || !seqused_cmp_kv || !cmp_residual_kv ||
      !ori_topk_length || !sinks || !attention_out)
    return AFA_E_NULL;
  const SparseArgs a = make_args(params, q, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table,
                                 cmp_block_table, cu_seqlens_q, seqused_ori_kv, seqused_cmp_kv,
                                 cmp_residual_kv, ori_topk_length, sinks, attention_out);
  hipStream_t s = (hipStream_t)stream;
  return params->dtype == AFA_DTYPE_BF16 ? dispatch_d<DT_BF16>(a, s) : dispatch_d<DT_F16>(a, s);
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

extern "C" int kernel_config_sparse_mla(int64_t cfg[5]) {
  if (!cfg) return AFA_E_NULL;
  cfg[0] = 13;  // external tensors
  cfg[1] = 0;   // runtime size parameters: all sizes travel in SparseMlaParams
  cfg[2] = 0;   // no workspace
  cfg[3] = 256; // MI355X compute units
  cfg[4] = 4;   // SIMDs per compute unit
  return AFA_OK;
}

extern "C" int workspace_size_sparse_mla(uint64_t* bytes, const SparseMlaParams* params) {
  if (!bytes) return -1;
  (void)params;
  *bytes = 0;
  return AFA_OK;
}

extern "C" const char* kernel_metadata_sparse_mla(void) {
  return "{\"version\":1,\"kernel\":\"sparse_mla\",\"tensors\":["
         "{\"name\":\"q\",\"dtype\":\"DTYPE\",\"shape\":[\"T\",\"H\",\"D\"],\"access\":\"read\"},"
         "{\"name\":\"ori_kv\",\"dtype\":\"DTYPE\",\"shape\":[\"ORI_BLOCKS\",\"PAGE\",1,\"D\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"cmp_kv\",\"dtype\":\"DTYPE\",\"shape\":[\"CMP_BLOCKS\",\"PAGE/RATIO\",1,\"D\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"cmp_sparse_indices\",\"dtype\":\"i32\",\"shape\":[\"T\",1,\"TOPK\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"ori_block_table\",\"dtype\":\"i32\",\"shape\":[\"B\",\"MAX_SEQ/PAGE\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"cmp_block_table\",\"dtype\":\"i32\",\"shape\":[\"B\",\"MAX_SEQ/PAGE\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"cu_seqlens_q\",\"dtype\":\"i32\",\"shape\":[\"B+1\"],\"access\":\"read\"},"
         "{\"name\":\"seqused_ori_kv\",\"dtype\":\"i32\",\"shape\":[\"B\"],\"access\":\"read\"},"
         "{\"name\":\"seqused_cmp_kv\",\"dtype\":\"i32\",\"shape\":[\"B\"],\"access\":\"read\"},"
         "{\"name\":\"cmp_residual_kv\",\"dtype\":\"i32\",\"shape\":[\"B\"],\"access\":\"read\"},"
         "{\"name\":\"ori_topk_length\",\"dtype\":\"i32\",\"shape\":[\"T\",1],\"access\":\"read\"},"
         "{\"name\":\"sinks\",\"dtype\":\"f32\",\"shape\":[\"H\"],\"access\":\"read\"},"
         "{\"name\":\"attention_out\",\"dtype\":\"DTYPE\",\"shape\":[\"T\",\"H\",\"D\"],"
         "\"access\":\"write\"}],"
         "\"parameters\":\"SparseMlaParams\",\"disjoint_external\":true,\"workspace\":false}";
}
