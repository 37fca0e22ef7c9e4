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

// query_metadata (gather.py:8-35) and the compressed bound (attention.py:339-341).
__device__ __forceinline__ Geometry token_geometry(const SparseArgs& a, int token) {
  int lo = 0, n = a.B;  // largest b in [0, B) with cu[b] <= token
  while (n > 1) {
    const int half = n >> 1;
    if (a.cu[lo + half] <= token) {
      lo += half;
      n -= half;
    } else {
      n = half;
    }
  }
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

// HG 16-head groups per workgroup (BM = 16*HG) and DS feature parts per head
// group: wave w owns heads 16*(w % HG) and features [w / HG * D/DS, +D/DS).
// With DS = 2 the two waves of a head group add their partial scores through
// LDS, so each wave keeps only half of Q and half of O in registers.
template <int DT, int D, int HG, int DS>
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
  static_assert(CHUNK * UNITS % NT == 0, "chunk must split evenly over the block");
  static_assert(UNITS >= 16, "swizzle needs at least 16 units per row");
  static_assert(DP % 32 == 0, "feature part must hold whole k-steps");

  __shared__ __attribute__((aligned(16))) uint8_t kv_lds[2][CHUNK * ROW_BYTES];
  __shared__ __attribute__((aligned(16))) f32x4 s_xchg[DS > 1 ? NW : 1][2][64];
  __shared__ int wave_count[NW];
  extern __shared__ uint32_t row_list[];  // round_up(WINDOW + TOPK, CHUNK) entries

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, i16 = lane & 15;
  const int hg = wave % HG, part = wave / HG;
  const int head_tiles = a.H / a.BM;
  const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
  const int token = (int)(logical / head_tiles);
  const int head0 = (int)(logical % head_tiles) * a.BM;

  const Geometry geo = token_geometry(a, token);

  // ---- 1. compact the selected rows into the LDS row list -------------------
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

  // ---- 2. Q fragments (B operand of S^T = KV * Q^T) for this wave's features
  const int head = head0 + hg * 16 + i16;
  const int dbase = part * DP;
  const scalar* q_row = (const scalar*)a.q + ((size_t)token * a.H + head) * D + dbase + 8 * g;
  x8 qf[DP / 32];
#pragma unroll
  for (int j = 0; j < DP / 32; ++j) qf[j] = *(const x8*)(q_row + 32 * j);

  f32x4 o[DP / 16];
#pragma unroll
  for (int t = 0; t < DP / 16; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  float m_run = a.sinks[head] * LOG2E;  // sink seeds the running max
  float l_run = g == 0 ? 1.0f : 0.0f;   // e^(sink - m) counted once per head
  const float scale_log2 = a.scale * LOG2E;

  // ---- 3. chunk loop: global -> registers -> LDS, then QK, softmax, PV ------
  u32x4 pf[PIECES];
  const char* ori = (const char*)a.ori_kv;
  const char* cmp = (const char*)a.cmp_kv;
  auto fetch = [&](int chunk) {
#pragma unroll
    for (int p = 0; p < PIECES; ++p) {
      const int flat = tid + p * NT;
      const int r = flat / UNITS, u = flat % UNITS;
      const uint32_t e = row_list[chunk * CHUNK + r];
      const char* base = (e & CMP_BIT) ? cmp : ori;
      pf[p] = *(const u32x4*)(base + (size_t)(e & ~CMP_BIT) * ROW_BYTES + u * 16);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PIECES; ++p) {
      const int flat = tid + p * NT;
      const int r = flat / UNITS, u = flat % UNITS;
      *(u32x4*)(&kv_lds[buf][r * ROW_BYTES + (swz(r, u) << 4)]) = pf[p];
    }
  };

  const int ra = sigma(i16);              // QK fragment row inside a 16-row tile
  const int rt = sigma(4 * g + (i16 >> 2));  // transposing-read row inside a tile
  const int tr_half = (i16 & 1) * 8;
  const int tr_unit = (i16 & 3) >> 1;
  const int ubase = dbase / 8;            // first 16-byte unit of this wave's features

  if (chunks > 0) fetch(0);
  for (int c = 0; c < chunks; ++c) {
    const int buf = c & 1;
    stash(buf);
    __syncthreads();
    if (c + 1 < chunks) fetch(c + 1);
    const uint8_t* tile = kv_lds[buf];

    // Partial S^T tiles over this wave's features, two chains per row tile.
    f32x4 s0a = {0.f, 0.f, 0.f, 0.f}, s0b = s0a, s1a = s0a, s1b = s0a;
#pragma unroll
    for (int j = 0; j < DP / 32; j += 2) {
      const int u0 = ubase + 4 * j + g, u1 = u0 + 4;
      const x8 a00 = *(const x8*)(tile + ra * ROW_BYTES + (swz(ra, u0) << 4));
      const x8 a10 = *(const x8*)(tile + (16 + ra) * ROW_BYTES + (swz(16 + ra, u0) << 4));
      const x8 a01 = *(const x8*)(tile + ra * ROW_BYTES + (swz(ra, u1) << 4));
      const x8 a11 = *(const x8*)(tile + (16 + ra) * ROW_BYTES + (swz(16 + ra, u1) << 4));
      s0a = B16<DT>::mfma(a00, qf[j], s0a);
      s1a = B16<DT>::mfma(a10, qf[j], s1a);
      s0b = B16<DT>::mfma(a01, qf[j + 1], s0b);
      s1b = B16<DT>::mfma(a11, qf[j + 1], s1b);
    }
    f32x4 s0 = s0a + s0b, s1 = s1a + s1b;
    if constexpr (DS > 1) {
      // Add the partner wave's partial scores (same heads, other features).
      // Both waves form own + partner in the same commutative pair, so they
      // hold bit-identical scores and take identical softmax decisions.
      s_xchg[wave][0][lane] = s0;
      s_xchg[wave][1][lane] = s1;
      __syncthreads();
      const int partner = (wave + HG) % NW;
      s0 += s_xchg[partner][0][lane];
      s1 += s_xchg[partner][1][lane];
    }

    // Online softmax for head `head`; this lane holds the chunk rows
    // sigma(4g+i) and 16 + sigma(4g+i).
    const int live = n_rows - c * CHUNK;
    float x0[4], x1[4];
    float cmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = sigma(4 * g + i);
      x0[i] = (row < live) ? s0[i] * scale_log2 : -INFINITY;
      x1[i] = (16 + row < live) ? s1[i] * scale_log2 : -INFINITY;
      cmax = fmaxf(cmax, fmaxf(x0[i], x1[i]));
    }
    cmax = max_over_lane_groups(cmax);
    const float m_new = fmaxf(m_run, cmax);
    if (c == 0) {
      l_run *= fast_exp2(m_run - m_new);  // O is still zero
      m_run = m_new;
    } else if (__ballot(m_new > m_run + TAU) != 0ull) {
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < DP / 16; ++t) o[t] *= alpha;
      m_run = m_new;
    }
    float psum = 0.f;
    x8 pf8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p0 = fast_exp2(x0[i] - m_run);
      const float p1 = fast_exp2(x1[i] - m_run);
      psum += p0 + p1;
      pf8[i] = (scalar)p0;
      pf8[4 + i] = (scalar)p1;
    }
    l_run += psum;

    // O^T[d, heads] += V^T[d, rows] * P^T[rows, heads] over this wave's features.
#pragma unroll
    for (int t = 0; t < DP / 16; ++t) {
      const int u = ubase + 2 * t + tr_unit;
      const x4 lo = B16<DT>::read_tr(
          (const AFA_LDS void*)(tile + rt * ROW_BYTES + (swz(rt, u) << 4) + tr_half));
      const x4 hi = B16<DT>::read_tr(
          (const AFA_LDS void*)(tile + (16 + rt) * ROW_BYTES + (swz(16 + rt, u) << 4) + tr_half));
      const x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[t] = B16<DT>::mfma(v, pf8, o[t]);
    }
  }

  // ---- 4. normalise and store: this lane holds d = dbase + 16t + 4g + i.
  const float inv = 1.0f / sum_over_lane_groups(l_run);
  scalar* out_row = (scalar*)a.out + ((size_t)token * a.H + head) * D + dbase + 4 * g;
#pragma unroll
  for (int t = 0; t < DP / 16; ++t) {
    x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (scalar)(o[t][i] * inv);
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
  const Geometry geo = token_geometry(a, token);
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

template <int DT, int D, int HG, int DS>
static int launch_fused(const SparseArgs& a, hipStream_t stream) {
  const int list = (a.WINDOW + a.TOPK + CHUNK - 1) / CHUNK * CHUNK;
  const size_t lds = (size_t)list * sizeof(uint32_t);
  const unsigned blocks = (unsigned)a.T * (unsigned)(a.H / a.BM);
  hipLaunchKernelGGL((sparse_mla_kernel<DT, D, HG, DS>), dim3(blocks), dim3(HG * DS * 64), lds,
                     stream, a);
  return (int)hipGetLastError();
}

template <int DT>
static int dispatch_d(const SparseArgs& a, hipStream_t s) {
  const bool four = a.BM == 64;
  switch (a.D) {
    case 128: return four ? launch_fused<DT, 128, 4, 1>(a, s) : launch_fused<DT, 128, 2, 1>(a, s);
    case 256: return four ? launch_fused<DT, 256, 4, 2>(a, s) : launch_fused<DT, 256, 2, 2>(a, s);
    default: return four ? launch_fused<DT, 512, 4, 2>(a, s) : launch_fused<DT, 512, 2, 2>(a, s);
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
