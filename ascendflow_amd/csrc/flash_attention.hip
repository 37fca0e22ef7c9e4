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


// KC keys per LDS stage; NW waves; QT 16-row query tiles per wave; D = 128.
template <int DT, int D, int NW, int QT, int KC>
__global__ __launch_bounds__(NW * 64) void fa_forward_kernel(FaArgs a) {
  typedef typename B16<DT>::scalar scalar;
  typedef typename B16<DT>::x8 x8;
  typedef typename B16<DT>::x4 x4;
  constexpr int NT = NW * 64;
  constexpr int UNITS = D / 8;
  constexpr int ROW_BYTES = D * 2;
  constexpr int PIECES = KC * UNITS / NT;  // per tensor (K and V) per thread
  constexpr int KT = KC / 16;              // key tiles per chunk
  constexpr int BQ = NW * QT * 16;         // query rows per workgroup
  static_assert(KC * UNITS % NT == 0, "chunk must split evenly");
  static_assert(KC % 32 == 0, "chunk must hold whole PV k-steps");

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[2][KC * ROW_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds[2][KC * ROW_BYTES];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, i16 = lane & 15;
  const int64_t q_tiles = (a.Sq + BQ - 1) / BQ;
  const uint32_t logical = xcd_contiguous(blockIdx.x, gridDim.x);
  // Causal: give the longest tiles (largest query rows) the lowest ids.
  int64_t qtile = (int64_t)(logical % q_tiles);
  if (a.causal) qtile = q_tiles - 1 - qtile;
  const int64_t bh = logical / q_tiles;
  const int head = (int)(bh % a.HQ), batch = (int)(bh / a.HQ);
  const int kv_head = head / (a.HQ / a.HKV);
  const int64_t q0 = qtile * BQ;

  const scalar* Q = (const scalar*)a.q + ((int64_t)batch * a.HQ + head) * a.Sq * D;
  const scalar* K = (const scalar*)a.k + ((int64_t)batch * a.HKV + kv_head) * a.Sk * D;
  const scalar* V = (const scalar*)a.v + ((int64_t)batch * a.HKV + kv_head) * a.Sk * D;
  scalar* O = (scalar*)a.o + ((int64_t)batch * a.HQ + head) * a.Sq * D;

  // Q fragments: B operand of S^T = K * Q^T. Query row of tile qt: q0 + wave*QT*16 + qt*16 + i16.
  x8 qf[QT][D / 32];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int64_t row = q0 + (wave * QT + qt) * 16 + i16;
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      if (row < a.Sq) {
        qf[qt][j] = *(const x8*)(Q + row * D + 32 * j + 8 * g);
      } else {
        qf[qt][j] = __builtin_bit_cast(x8, u32x4{0u, 0u, 0u, 0u});
      }
    }
  }
  f32x4 o[QT][D / 16];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) o[qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float scale_log2 = a.scale * FA_LOG2E;

  int64_t kv_end = a.Sk;
  if (a.causal) kv_end = min(a.Sk, q0 + BQ);  // keys beyond the tile's last query are masked
  const int chunks = (int)((kv_end + KC - 1) / KC);

  u32x4 pk[PIECES], pv[PIECES];
  auto fetch = [&](int chunk) {
#pragma unroll
    for (int p = 0; p < PIECES; ++p) {
      const int flat = tid + p * NT, r = flat / UNITS, u = flat % UNITS;
      const int64_t key = (int64_t)chunk * KC + r;
      if (key < a.Sk) {
        pk[p] = *(const u32x4*)(K + key * D + u * 8);
        pv[p] = *(const u32x4*)(V + key * D + u * 8);
      } else {
        pk[p] = u32x4{0u, 0u, 0u, 0u};
        pv[p] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PIECES; ++p) {
      const int flat = tid + p * NT, r = flat / UNITS, u = flat % UNITS;
      const int off = r * ROW_BYTES + (swz(r, u) << 4);
      *(u32x4*)(&k_lds[buf][off]) = pk[p];
      *(u32x4*)(&v_lds[buf][off]) = pv[p];
    }
  };

  const int ra = sigma(i16);
  const int rt = sigma(4 * g + (i16 >> 2));
  const int tr_half = (i16 & 1) * 8, tr_unit = (i16 & 3) >> 1;

  if (chunks > 0) fetch(0);
  for (int c = 0; c < chunks; ++c) {
    const int buf = c & 1;
    stash(buf);
    __syncthreads();
    if (c + 1 < chunks) fetch(c + 1);
    const uint8_t* kt = k_lds[buf];
    const uint8_t* vt = v_lds[buf];
    const int64_t key0 = (int64_t)c * KC;

    // S^T[key tile kt_][query tile qt].
    f32x4 s[KT][QT];
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[t][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      const int u = 4 * j + g;
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const int row = 16 * t + ra;
        const x8 kf = *(const x8*)(kt + row * ROW_BYTES + (swz(row, u) << 4));
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) s[t][qt] = B16<DT>::mfma(kf, qf[qt][j], s[t][qt]);
      }
    }

    // Online softmax per query tile; this lane holds query q (column i16) and
    // keys key0 + 16t + sigma(4g + i).
    x8 pf[QT][KC / 32];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int64_t query = q0 + (wave * QT + qt) * 16 + i16;
      float x[KT][4];
      float cmax = -INFINITY;
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t key = key0 + 16 * t + sigma(4 * g + i);
          const bool ok = key < a.Sk && (!a.causal || key <= query);
          x[t][i] = ok ? s[t][qt][i] * scale_log2 : -INFINITY;
          cmax = fmaxf(cmax, x[t][i]);
        }
      cmax = max_over_lane_groups(cmax);
      const float m_new = fmaxf(m_run[qt], cmax);
      const float base = m_new == -INFINITY ? 0.f : m_new;  // fully masked so far
      const float alpha = fast_exp2(m_run[qt] - base);
      m_run[qt] = m_new;
      float psum = 0.f;
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(x[t][i] - base);
          psum += p;
          pf[qt][t >> 1][(t & 1) * 4 + i] = (scalar)p;
        }
      l_run[qt] = l_run[qt] * alpha + psum;
#pragma unroll
      for (int t = 0; t < D / 16; ++t) o[qt][t] *= alpha;
    }

    // O^T[d, q] += V^T[d, keys] * P^T[keys, q].
#pragma unroll
    for (int ks = 0; ks < KC / 32; ++ks) {
#pragma unroll
      for (int t = 0; t < D / 16; ++t) {
        const int u = 2 * t + tr_unit;
        const int r0 = 32 * ks + rt, r1 = 32 * ks + 16 + rt;
        const x4 lo = B16<DT>::read_tr(
            (const AFA_LDS void*)(vt + r0 * ROW_BYTES + (swz(r0, u) << 4) + tr_half));
        const x4 hi = B16<DT>::read_tr(
            (const AFA_LDS void*)(vt + r1 * ROW_BYTES + (swz(r1, u) << 4) + tr_half));
        const x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][t] = B16<DT>::mfma(vf, pf[qt][ks], o[qt][t]);
      }
    }
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
constexpr int FA_NW = 4, FA_QT = 2, FA_KC = 64;

template <int DT>
int launch_fa(const FaArgs& a, hipStream_t s) {
  constexpr int BQ = FA_NW * FA_QT * 16;
  const int64_t tiles = (a.Sq + BQ - 1) / BQ;
  const int64_t blocks = tiles * a.B * a.HQ;
  if (blocks > 0x7fffffffLL) return AFA_E_SHAPE;
  hipLaunchKernelGGL((fa_forward_kernel<DT, 128, FA_NW, FA_QT, FA_KC>), dim3((unsigned)blocks),
                     dim3(FA_NW * 64), 0, s, a);
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

extern "C" const char* kernel_metadata_attention_target(void) {
  return "{\"version\":1,\"kernel\":\"attention_target\",\"tensors\":["
         "{\"name\":\"Q\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HQ\",\"Sq\",\"D\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"K\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HKV\",\"Sk\",\"D\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"V\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HKV\",\"Sk\",\"D\"],"
         "\"access\":\"read\"},"
         "{\"name\":\"O\",\"dtype\":\"DTYPE\",\"shape\":[\"B\",\"HQ\",\"Sq\",\"D\"],"
         "\"access\":\"write\"}],"
         "\"parameters\":[{\"name\":\"Sq\",\"minimum\":1},{\"name\":\"Sk\",\"minimum\":1}],"
         "\"disjoint_external\":true,\"workspace\":false}";
}

extern "C" const char* kernel_metadata_simple_attention(void) {
  return "{\"version\":1,\"kernel\":\"simple_attention\",\"tensors\":["
         "{\"name\":\"Q\",\"dtype\":\"f16\",\"shape\":[\"H\",\"S\",128],\"access\":\"read\"},"
         "{\"name\":\"K\",\"dtype\":\"f16\",\"shape\":[\"H\",128,128],\"access\":\"read\"},"
         "{\"name\":\"V\",\"dtype\":\"f16\",\"shape\":[\"H\",128,128],\"access\":\"read\"},"
         "{\"name\":\"O\",\"dtype\":\"f16\",\"shape\":[\"H\",\"S\",128],\"access\":\"write\"}],"
         "\"parameters\":[{\"name\":\"S\",\"minimum\":64,\"multiple\":64},"
         "{\"name\":\"H\",\"minimum\":1}],\"disjoint_external\":true,\"workspace\":false}";
}
