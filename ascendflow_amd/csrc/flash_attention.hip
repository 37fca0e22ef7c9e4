// Flash attention forward (BNSD) and the teaching single-tile attention for
// gfx950.
//
// attention_target: examples/flash_attention/attention.py:243-417. The
// reference's Cube/Vector stages (QK -> Score GM -> online softmax -> P GM ->
// PV -> PV GM -> rescale/update) collapse into one kernel per (batch, head,
// query tile): K and V chunks stream through double-buffered, XOR-swizzled
// LDS; each wave owns QT*16 query rows with Q resident in registers;
// S^T[keys, queries] = K * Q^T and O^T[d, queries] += V^T * P^T run on
// v_mfma_f32_16x16x32_{f16,bf16}; the online softmax (attention.py:73-139:
// m' = max(m, rowmax s), alpha = e^(m-m'), l = l*alpha + sum p, O = O*alpha +
// b16(p) V) stays in FP32 registers; V^T fragments come through
// ds_read_b64_tr_b16. Causal masking is top-left (key j visible to query i iff
// j <= i, attention.py:96-110); keys >= Sk and queries >= Sq are masked.
//
// simple_attention: examples/flash_attention/simple.py:60-141. One 128-key
// tile per head: S = Q K^T * 128^-1/2, P = f16(softmax(S)) normalised BEFORE
// the cast, O = f16(P V) (simple.py:25-57).
#include "common.h"
#include "../../include/ascendflow_amd.h"

namespace afa {

constexpr float FA_LOG2E = 1.4426950408889634f;

struct FaArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t Sq, Sk;
  int32_t B, HQ, HKV, causal;
  float scale;
};


// Flash-attention forward for D = 128. One workgroup of NW waves owns BQ =
// NW * QT * 16 query rows of one (batch, head); each wave owns QT 16-row query
// tiles with Q resident in registers. K and V stream in KC-key chunks through
// a 3-stage LDS ring filled by the load-to-LDS path two chunks ahead (rows
// XOR-swizzled on the global side, unit u of row r at u ^ (r & 15)).
// S^T[keys, queries] = K * Q^T and O^T[d, queries] += V^T * P^T run on
// v_mfma_f32_16x16x32_{f16,bf16}; V^T fragments come through
// ds_read_b64_tr_b16. Per chunk c the QK MFMAs of chunk c + 1 are issued
// ahead of the softmax of chunk c, so they run under its VALU work.
//
// Online softmax (attention.py:73-139) in FP32 registers, exp2 domain: the
// chunk max is taken on raw scores (the scale is positive) and the scale goes
// into the exponent's FMA; the running max is raised, with O and l rescaled
// by alpha = 2^(m - m'), only when some query's max exceeds it by more than
// fa_tau, so P <= 2^fa_tau; O / l is independent of the reference point. The
// lazy reference point rounds the P of the key holding the running max to the
// storage dtype, where the reference's recurrence has P = 1 exactly: a
// relative error of at most 2^-12 in f16 (within its contract; eager rescaling
// measured 5% slower on FA C2) but 2^-9 in bf16, which with sharp scores moved
// outputs by 2 ulps, so bf16 raises the max whenever it grows (fa_tau = 0).
// Masks (attention.py:96-110): keys >= Sk, and for causal attention key j is
// visible to query i iff j <= i (top-left); they are applied only in chunks
// that reach the tail or the diagonal.
template <int DT> __device__ constexpr float fa_tau() { return DT == DT_F16 ? 8.0f : 0.0f; }
constexpr int FA_NSTAGE = 3;
// Progress-ordered wave priorities: a wave starts each chunk at priority 3
// and steps down at half of QK, after QK and at half of PV, so of the two waves
// sharing a SIMD the one behind wins the MFMA arbitration (otherwise the older
// wave always wins, finishes first and waits at the barrier while the other
// runs alone).
constexpr bool FA_PROGRESS_PRIO = true;

template <int DT, int NW, int QT>
__global__ __launch_bounds__(NW * 64) void fa_forward_kernel(FaArgs a) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x8 x8;
  typedef typename B16<DT>::x4 x4;
  constexpr int D = 128, ROW_BYTES = 2 * D, UNITS = D / 8;
  constexpr int KC = 64;                       // keys per chunk
  constexpr int KT = KC / 16;                  // key tiles per chunk
  constexpr int TILE = KC * ROW_BYTES;         // bytes of one K or V tile
  constexpr int BQ = NW * QT * 16;
  constexpr int ROWS_PER_LOAD = 64 / UNITS;    // rows one wave load covers
  constexpr int LOADS = KC / ROWS_PER_LOAD / NW;  // wave loads per tensor per chunk
  static_assert(LOADS * ROWS_PER_LOAD * NW == KC, "a chunk must split evenly over the waves");

  __shared__ __attribute__((aligned(16))) uint8_t kv_lds[FA_NSTAGE][2][TILE];  // [stage][K, V]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 4, i16 = lane & 15;
  const int64_t q_tiles = (a.Sq + BQ - 1) / BQ;
  const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
  // Causal: the longest tiles (largest query rows) get the lowest ids.
  int64_t qtile = (int64_t)(logical % q_tiles);
  if (a.causal) qtile = q_tiles - 1 - qtile;
  const int64_t bh = logical / q_tiles;
  const int head = (int)(bh % a.HQ), batch = (int)(bh / a.HQ);
  const int kv_head = head / (a.HQ / a.HKV);
  const int64_t q0 = qtile * BQ;

  const scalar* Q = (const scalar*)a.q + ((int64_t)batch * a.HQ + head) * a.Sq * D;
  const char* K = (const char*)a.k + ((int64_t)batch * a.HKV + kv_head) * a.Sk * ROW_BYTES;
  const char* V = (const char*)a.v + ((int64_t)batch * a.HKV + kv_head) * a.Sk * ROW_BYTES;
  scalar* O = (scalar*)a.o + ((int64_t)batch * a.HQ + head) * a.Sq * D;

  // Q fragments: B operand of S^T = K * Q^T; query of tile qt: q0 + (wave*QT + qt)*16 + i16.
  x8 qf[QT][D / 32];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int64_t row = q0 + (wave * QT + qt) * 16 + i16;
#pragma unroll
    for (int j = 0; j < D / 32; ++j)
      qf[qt][j] = row < a.Sq ? *(const x8*)(Q + row * D + 32 * j + 8 * g) : __builtin_bit_cast(x8, u32x4{0u, 0u, 0u, 0u});
  }

  int64_t kv_end = a.Sk;
  if (a.causal) kv_end = min(a.Sk, q0 + BQ);  // keys past the tile's last query are masked
  const int chunks = (int)((kv_end + KC - 1) / KC);
  // First chunk that needs masking: it reaches Sk or (causal) the tile's first query.
  int64_t clean_end = a.Sk;
  if (a.causal) clean_end = min(clean_end, q0 + 1);
  const int clean_chunks = (int)(clean_end / KC);

  // ---- KV movement ---------------------------------------------------------
  const uint32_t kv_base = lds_address(kv_lds[0][0]);
  auto tile_address = [&](int chunk, int tensor) {
    return opaque_uniform(kv_base + (uint32_t)((chunk % FA_NSTAGE) * 2 + tensor) * TILE);
  };
  // Wave load p of a chunk covers rows [(wave*LOADS + p)*ROWS_PER_LOAD, +ROWS_PER_LOAD);
  // this lane lands on unit (lane % UNITS) of row lane / UNITS and loads unit
  // (lane % UNITS) ^ (row & 15) of that row.
  uint32_t load_offset[LOADS];
#pragma unroll
  for (int p = 0; p < LOADS; ++p) {
    const int r = (wave * LOADS + p) * ROWS_PER_LOAD + lane / UNITS;
    load_offset[p] = (uint32_t)(r * ROW_BYTES + (((lane % UNITS) ^ (r & 15)) << 4));
  }
  auto fetch = [&](int chunk) {
    const int64_t key0 = (int64_t)chunk * KC;
    const char* kbase = K + key0 * ROW_BYTES;
    const char* vbase = V + key0 * ROW_BYTES;
    const bool tail = key0 + KC > a.Sk;
#pragma unroll
    for (int p = 0; p < LOADS; ++p) {
      uint32_t off = load_offset[p];
      if (tail) {  // rows past Sk read the last key instead (masked later)
        const int r = (wave * LOADS + p) * ROWS_PER_LOAD + lane / UNITS;
        const int rr = (int)min((int64_t)r, a.Sk - 1 - key0);
        off = (uint32_t)(rr * ROW_BYTES + (((lane % UNITS) ^ (r & 15)) << 4));
      }
      const uint32_t row0 = (uint32_t)((wave * LOADS + p) * ROWS_PER_LOAD * ROW_BYTES);
      const uint32_t kd = tile_address(chunk, 0) + row0, vd = tile_address(chunk, 1) + row0;
      __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                       :: "s"(kd), "v"(off), "s"(kbase) : "memory");
      __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                       :: "s"(vd), "v"(off), "s"(vbase) : "memory");
    }
  };

  // ---- fragment addressing ---------------------------------------------------
  const int ra = sigma(i16);                 // K fragment row inside a 16-key tile
  const int rt = sigma(4 * g + (i16 >> 2));  // transposing-read row inside a tile
  uint32_t qk_base[D / 32], tr_base[D / 16];
#pragma unroll
  for (int j = 0; j < D / 32; ++j) qk_base[j] = (uint32_t)(ra * ROW_BYTES + (((4 * j + g) ^ (ra & 15)) << 4));
#pragma unroll
  for (int t = 0; t < D / 16; ++t)
    tr_base[t] = (uint32_t)(rt * ROW_BYTES + (((2 * t + ((i16 & 3) >> 1)) ^ (rt & 15)) << 4) + (i16 & 1) * 8);

  f32x4 o[QT][D / 16];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -1e30f;  // finite: a fully masked chunk then gives p = 0, never NaN
    l_run[qt] = 0.f;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) o[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float scale_log2 = a.scale * FA_LOG2E;

  // S^T of one chunk: K fragments LOOK steps ahead of their MFMAs. After the
  // MFMAs of fragment f, between(f) issues independent VALU work (the softmax
  // of the previous chunk), which runs in the shadow of the MFMA pipe.
  constexpr int QK_FRAGS = (D / 32) * KT;  // 16 fragments, each feeds QT MFMAs
  constexpr int LOOK = 6;
  auto qk_chunk = [&](int chunk, f32x4 (&s)[KT][QT], auto&& between) {
    const uint32_t tile = tile_address(chunk, 0);
    uint32_t base[D / 32];
#pragma unroll
    for (int j = 0; j < D / 32; ++j) base[j] = opaque(tile + qk_base[j]);
    x8 kf[QK_FRAGS];
    auto load = [&](int f) {  // fragment f = (j, t): k-step j, key tile t
      const int j = f / KT, t = f % KT;
      kf[f] = *(const AFA_LDS x8*)(lds_at<uint8_t>(base[j]) + t * 16 * ROW_BYTES);
    };
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[t][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int f = 0; f < LOOK && f < QK_FRAGS; ++f) load(f);
#pragma unroll
    for (int f = 0; f < QK_FRAGS; ++f) {
      if (f + LOOK < QK_FRAGS) load(f + LOOK);
      const int j = f / KT, t = f % KT;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[t][qt] = B16<DT>::mfma(kf[f], qf[qt][j], s[t][qt]);
      between(f);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // O^T[d, q] += V^T[d, keys] * P^T[keys, q], with between(f) as in qk_chunk.
  constexpr int PV_FRAGS = (KC / 32) * (D / 16);  // 16 fragments, each feeds QT MFMAs
  auto pv_chunk = [&](int chunk, x8 (&pf)[QT][KC / 32], auto&& between) {
    const uint32_t tile = tile_address(chunk, 1);
    uint32_t vb[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; ++t) vb[t] = opaque(tile + tr_base[t]);
    constexpr int VLOOK = 3;
    x4 vlo[PV_FRAGS], vhi[PV_FRAGS];
    auto vload = [&](int f) {  // f = (ks, t)
      const int ks = f / (D / 16), t = f % (D / 16);
      const AFA_LDS uint8_t* p = lds_at<uint8_t>(vb[t]) + ks * 32 * ROW_BYTES;
      vlo[f] = B16<DT>::read_tr((const AFA_LDS void*)p);
      vhi[f] = B16<DT>::read_tr((const AFA_LDS void*)(p + 16 * ROW_BYTES));
    };
#pragma unroll
    for (int f = 0; f < VLOOK; ++f) vload(f);
#pragma unroll
    for (int f = 0; f < PV_FRAGS; ++f) {
      if (f + VLOOK < PV_FRAGS) vload(f + VLOOK);
      const int ks = f / (D / 16), t = f % (D / 16);
      const x8 vf = {vlo[f][0], vlo[f][1], vlo[f][2], vlo[f][3], vhi[f][0], vhi[f][1], vhi[f][2], vhi[f][3]};
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) o[qt][t] = B16<DT>::mfma(vf, pf[qt][ks], o[qt][t]);
      between(f);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Scores of keys at or past a per-column limit (the tail chunk and the
  // causal diagonal) become -inf; 32-bit chunk-relative indices. This lane
  // holds query (column) i16 of each query tile and keys 16t + sigma(4g + i).
  auto mask = [&](int chunk, f32x4 (&s)[KT][QT]) {
    const int64_t key0 = (int64_t)chunk * KC;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int64_t query = q0 + (wave * QT + qt) * 16 + i16;
      int64_t limit = a.Sk - key0;
      if (a.causal) limit = limit < query - key0 + 1 ? limit : query - key0 + 1;
      const int lim = limit < 0 ? 0 : (limit > KC ? KC : (int)limit);
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[t][qt][i] = 16 * t + sigma(4 * g + i) < lim ? s[t][qt][i] : -INFINITY;
    }
  };

  // ---- pipeline: chunk c+2 loads, QK(c+1) + softmax(c), PV(c) + softmax(c) --
  // Chunk c's scores are in cur (masked at the top of its iteration) and
  // QK(c+1) writes nxt; the loop is unrolled by two so the two score buffers
  // alternate without copies. The softmax of chunk c is spread over the MFMA
  // steps: the first QT steps of QK(c+1) take the column maxima, the next two
  // the cross-lane reduction and the (rare, uniform) rescale, the rest the
  // exponentials of key tiles 0-1; the first PV(c) steps, which use only
  // those, take the exponentials of key tiles 2-3.
  constexpr int HALF = QT * 8;                  // exponentials per key-tile pair
  constexpr int QK_EXP0 = QT + 2;               // first QK step with exponentials
  constexpr int PV_EXP_STEPS = PV_FRAGS / 2 - 1;  // PV steps with exponentials
  static_assert(QK_FRAGS > QK_EXP0, "no QK step left for exponentials");
  f32x4 s_a[KT][QT], s_b[KT][QT];
  if (chunks > 0) fetch(0);
  if (chunks > 1) fetch(1);
  if (chunks > 0) {
    if (chunks > 1)
      __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * LOADS));  // KV(0) landed, KV(1) may be in flight
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);
    block_barrier();
    qk_chunk(0, s_a, [](int) {});
  }
  auto iteration = [&](int c, f32x4 (&cur)[KT][QT], f32x4 (&nxt)[KT][QT]) {
    // KV(c+1) landed (its loads are the only ones in flight); after the
    // barrier every wave is past PV(c-1), so tile (c+2) % 3 is free.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    block_barrier();
    if (c + 2 < chunks) fetch(c + 2);
    if (c >= clean_chunks) mask(c, cur);

    x8 pf[QT][KC / 32];
    float cmax[QT], m_new[QT], psum[QT];
    auto exp_element = [&](int e) {  // e = (half, qt, t & 1, i)
      const int h = e / HALF, qt = (e / 8) % QT, t = 2 * h + (e / 4) % 2, i = e % 4;
      const float p = fast_exp2(__builtin_fmaf(cur[t][qt][i], scale_log2, -m_run[qt]));
      psum[qt] += p;
      pf[qt][h][(t & 1) * 4 + i] = (scalar)p;
    };
    auto qk_between = [&](int f) {
      if (FA_PROGRESS_PRIO && f == QK_FRAGS / 2 - 1) __builtin_amdgcn_s_setprio(2);
      if (f < QT) {
        float m = -INFINITY;
#pragma unroll
        for (int t = 0; t < KT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) m = fmaxf(m, cur[t][f][i]);
        cmax[f] = m;
      } else if (f == QT) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          m_new[qt] = fmaxf(m_run[qt], max_over_lane_groups(cmax[qt]) * scale_log2);
          psum[qt] = 0.f;
        }
      } else if (f == QT + 1) {
        bool grow = false;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) grow |= m_new[qt] > m_run[qt] + fa_tau<DT>();
        if (__ballot(grow) != 0ull) {
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            const float alpha = fast_exp2(m_run[qt] - m_new[qt]);
            l_run[qt] *= alpha;
#pragma unroll
            for (int t = 0; t < D / 16; ++t) o[qt][t] *= alpha;
            m_run[qt] = m_new[qt];
          }
        }
      } else {
        // Constant trip counts: the loop unrolls before f is known.
#pragma unroll
        for (int e = 0; e < HALF; ++e)
          if (QK_EXP0 + e * (QK_FRAGS - QK_EXP0) / HALF == f) exp_element(e);
      }
    };
    auto pv_between = [&](int f) {
      if (FA_PROGRESS_PRIO && f == PV_FRAGS / 2 - 1) __builtin_amdgcn_s_setprio(0);
      if (f < PV_EXP_STEPS) {
#pragma unroll
        for (int e = 0; e < HALF; ++e)
          if (e * PV_EXP_STEPS / HALF == f) exp_element(HALF + e);
      } else if (f == PV_EXP_STEPS + 1) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) l_run[qt] += psum[qt];
      }
    };

    // The last chunk also runs a QK, over the stale tile (c + 1) % 3 (no load
    // is in flight into it), so that the softmax has one code path; those
    // scores are never read.
    if (FA_PROGRESS_PRIO) __builtin_amdgcn_s_setprio(3);
    qk_chunk(c + 1, nxt, qk_between);
    if (FA_PROGRESS_PRIO) __builtin_amdgcn_s_setprio(1);
    pv_chunk(c, pf, pv_between);
  };
  for (int c = 0; c < chunks; c += 2) {
    iteration(c, s_a, s_b);
    if (c + 1 < chunks) iteration(c + 1, s_b, s_a);
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int64_t query = q0 + (wave * QT + qt) * 16 + i16;
    const float l = sum_over_lane_groups(l_run[qt]);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    if (query < a.Sq) {
      scalar* orow = O + query * D + 4 * g;
#pragma unroll
      for (int t = 0; t < D / 16; ++t) {
        x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (scalar)(o[qt][t][i] * inv);
        *(x4*)(orow + 16 * t) = v;
      }
    }
  }
}

// Teaching attention: one workgroup per (head, 64 query rows), 4 waves of 16
// queries; the whole 128-key tile is resident, so the softmax is exact and P
// is normalised before its f16 cast (simple.py:25-41).
__global__ __launch_bounds__(256) void simple_attention_kernel(const _Float16* Qp,
                                                               const _Float16* Kp,
                                                               const _Float16* Vp, _Float16* Op,
                                                               int64_t S) {
  typedef B16<DT_F16> ops;
  constexpr int D = 128, SK = 128, ROW_BYTES = D * 2, KT = SK / 16;
  __shared__ __attribute__((aligned(16))) uint8_t k_lds[SK * ROW_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds[SK * ROW_BYTES];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, i16 = lane & 15;
  const int64_t tiles = S / 64;
  const int64_t head = blockIdx.x / tiles, tile = blockIdx.x % tiles;
  const _Float16* Q = Qp + head * S * D;
  const _Float16* K = Kp + head * SK * D;
  const _Float16* V = Vp + head * SK * D;
  _Float16* O = Op + head * S * D;

  for (int flat = tid; flat < SK * (D / 8); flat += 256) {
    const int r = flat / (D / 8), u = flat % (D / 8);
    const int off = r * ROW_BYTES + (swz(r, u) << 4);
    *(u32x4*)(&k_lds[off]) = *(const u32x4*)(K + r * D + u * 8);
    *(u32x4*)(&v_lds[off]) = *(const u32x4*)(V + r * D + u * 8);
  }
  const int64_t query = tile * 64 + wave * 16 + i16;
  f16x8 qf[D / 32];
#pragma unroll
  for (int j = 0; j < D / 32; ++j) qf[j] = *(const f16x8*)(Q + query * D + 32 * j + 8 * g);
  __syncthreads();

  const int ra = sigma(i16);
  f32x4 s[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < D / 32; ++j) {
    const int u = 4 * j + g;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const int row = 16 * t + ra;
      const f16x8 kf = *(const f16x8*)(k_lds + row * ROW_BYTES + (swz(row, u) << 4));
      s[t] = ops::mfma(kf, qf[j], s[t]);
    }
  }
  const float scale_log2 = 0.08838834764831845f * FA_LOG2E;
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[t][i] *= scale_log2;
      mx = fmaxf(mx, s[t][i]);
    }
  mx = max_over_lane_groups(mx);
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[t][i] = fast_exp2(s[t][i] - mx);
      sum += s[t][i];
    }
  const float inv = 1.0f / sum_over_lane_groups(sum);
  f16x8 pf[SK / 32];
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) pf[t >> 1][(t & 1) * 4 + i] = (_Float16)(s[t][i] * inv);

  const int rt = sigma(4 * g + (i16 >> 2));
  const int tr_half = (i16 & 1) * 8, tr_unit = (i16 & 3) >> 1;
  _Float16* orow = O + query * D + 4 * g;
#pragma unroll
  for (int t = 0; t < D / 16; ++t) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int u = 2 * t + tr_unit;
#pragma unroll
    for (int ks = 0; ks < SK / 32; ++ks) {
      const int r0 = 32 * ks + rt, r1 = 32 * ks + 16 + rt;
      const f16x4 lo = ops::read_tr(
          (const AFA_LDS void*)(v_lds + r0 * ROW_BYTES + (swz(r0, u) << 4) + tr_half));
      const f16x4 hi = ops::read_tr(
          (const AFA_LDS void*)(v_lds + r1 * ROW_BYTES + (swz(r1, u) << 4) + tr_half));
      const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      acc = ops::mfma(vf, pf[ks], acc);
    }
    f16x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (_Float16)acc[i];
    *(f16x4*)(orow + 16 * t) = v;
  }
}

}  // namespace afa

using namespace afa;

namespace {
constexpr int FA_NW = 8, FA_QT = 2;

template <int DT>
int launch_fa(const FaArgs& a, hipStream_t s) {
  constexpr int BQ = FA_NW * FA_QT * 16;
  const int64_t tiles = (a.Sq + BQ - 1) / BQ;
  const int64_t blocks = tiles * a.B * a.HQ;
  if (blocks > 0x7fffffffLL) return AFA_E_SHAPE;
  hipLaunchKernelGGL((fa_forward_kernel<DT, FA_NW, FA_QT>), dim3((unsigned)blocks), dim3(FA_NW * 64), 0, s, a);
  return (int)hipGetLastError();
}
}  // namespace

extern "C" int launch_attention_target(void* stream, const void* Q, const void* K, const void* V,
                                       void* O, void* workspace, int64_t Sq, int64_t Sk,
                                       const FaParams* p) {
  (void)workspace;
  if (!p) return AFA_E_NULL;
  if (!Q || !K || !V || !O) return AFA_E_NULL;
  if (p->dtype != AFA_DTYPE_BF16 && p->dtype != AFA_DTYPE_F16) return AFA_E_DTYPE;
  if (p->D != 128 || p->B <= 0 || p->HQ <= 0 || p->HKV <= 0 || p->HQ % p->HKV) return AFA_E_SHAPE;
  if (Sq < 1 || Sk < 1 || !(p->scale > 0.0f)) return AFA_E_SHAPE;
  FaArgs a;
  a.q = Q;
  a.k = K;
  a.v = V;
  a.o = O;
  a.Sq = Sq;
  a.Sk = Sk;
  a.B = p->B;
  a.HQ = p->HQ;
  a.HKV = p->HKV;
  a.causal = p->causal ? 1 : 0;
  a.scale = p->scale;
  hipStream_t s = (hipStream_t)stream;
  return p->dtype == AFA_DTYPE_F16 ? launch_fa<DT_F16>(a, s) : launch_fa<DT_BF16>(a, s);
}

extern "C" int launch_simple_attention(void* stream, const void* Q, const void* K, const void* V,
                                       void* O, void* workspace, int64_t S, int64_t H) {
  (void)workspace;
  if (!Q || !K || !V || !O) return AFA_E_NULL;
  if (S <= 0 || S % 64 || H <= 0 || (S / 64) * H > 0x7fffffffLL) return AFA_E_SHAPE;
  hipLaunchKernelGGL(simple_attention_kernel, dim3((unsigned)((S / 64) * H)), dim3(256), 0,
                     (hipStream_t)stream, (const _Float16*)Q, (const _Float16*)K,
                     (const _Float16*)V, (_Float16*)O, S);
  return (int)hipGetLastError();
}

extern "C" int kernel_config_attention_target(int64_t cfg[5]) {
  if (!cfg) return AFA_E_NULL;
  cfg[0] = 4;
  cfg[1] = 2;  // Sq, Sk
  cfg[2] = 0;
  cfg[3] = 256;
  cfg[4] = 4;
  return AFA_OK;
}

extern "C" int kernel_config_simple_attention(int64_t cfg[5]) {
  if (!cfg) return AFA_E_NULL;
  cfg[0] = 4;
  cfg[1] = 2;  // S, H
  cfg[2] = 0;
  cfg[3] = 256;
  cfg[4] = 4;
  return AFA_OK;
}

extern "C" int workspace_size_attention_target(uint64_t* bytes, int64_t Sq, int64_t Sk,
                                               const FaParams* p) {
  if (!bytes) return -1;
  (void)Sq;
  (void)Sk;
  (void)p;
  *bytes = 0;
  return AFA_OK;
}

extern "C" int workspace_size_simple_attention(uint64_t* bytes, int64_t S, int64_t H) {
  if (!bytes) return -1;
  (void)S;
  (void)H;
  *bytes = 0;
  return AFA_OK;
}

// Launch-ABI descriptions in the reference's metadata schema
// (src/backend/abi.py:19-59): tensors (dtype, shape with named axes, layout,
// access), runtime size parameters with minimum and multiple, workspace flag.
// The FA sizes the reference specialises at compile time (B, HQ, HKV, D,
// dtype, causal, scale) travel in FaParams ("params_struct"); "DTYPE" is one
// of "dtypes".
extern "C" const char* kernel_metadata_attention_target(void) {
  return "{\"version\":1,\"name\":\"attention_target\",\"target\":\"gfx950\",\"kind\":\"mixed\","
         "\"groups\":256,\"disjoint_external\":true,\"device_resources\":null,"
         "\"dtypes\":{\"DTYPE\":[\"f16\",\"bf16\"]},\"tensors\":["
         "{\"name\":\"Q\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HQ\",\"Sq\",\"D\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"K\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HKV\",\"Sk\",\"D\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"V\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HKV\",\"Sk\",\"D\"],"
         "\"layout\":\"linear\",\"access\":\"read\"},"
         "{\"name\":\"O\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HQ\",\"Sq\",\"D\"],"
         "\"layout\":\"linear\",\"access\":\"write\"}],"
         "\"parameters\":[{\"name\":\"Sq\",\"minimum\":1,\"multiple\":1},"
         "{\"name\":\"Sk\",\"minimum\":1,\"multiple\":1}],"
         "\"params_struct\":{\"name\":\"FaParams\",\"fields\":[\"B\",\"HQ\",\"HKV\",\"D\",\"dtype\","
         "\"causal\",\"scale\",\"reserved\"]},"
         "\"workspace\":false}";
}
extern "C" const char* kernel_metadata_simple_attention(void) {
  return "{\"version\":1,\"name\":\"simple_attention\",\"target\":\"gfx950\",\"kind\":\"mixed\","
         "\"groups\":256,\"disjoint_external\":true,\"device_resources\":null,\"tensors\":["
         "{\"name\":\"Q\",\"dtype\":\"f16\",\"shape\":[\"H\",\"S\",128],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"K\",\"dtype\":\"f16\",\"shape\":[\"H\",128,128],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"V\",\"dtype\":\"f16\",\"shape\":[\"H\",128,128],\"layout\":\"linear\","
         "\"access\":\"read\"},"
         "{\"name\":\"O\",\"dtype\":\"f16\",\"shape\":[\"H\",\"S\",128],\"layout\":\"linear\","
         "\"access\":\"write\"}],"
         "\"parameters\":[{\"name\":\"S\",\"minimum\":64,\"multiple\":64},"
         "{\"name\":\"H\",\"minimum\":1,\"multiple\":1}],\"workspace\":false}";
}
