// Host-side checks of libascendflow_amd's C ABI, built with AddressSanitizer
// and UndefinedBehaviorSanitizer on the host code only (tests/test_host_sanitizers.py)
// and run on the CPU: every call here returns before any kernel launch or
// device query (validation, workspace sizing, the split cost model, metadata
// and config queries), so it needs no GPU. Exits non-zero when any expectation
// fails; the sanitizers abort on any memory or undefined-behaviour error.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "ascendflow_amd.h"

static int failures = 0;
#define EXPECT(cond)                                                 \
  do {                                                               \
    if (!(cond)) {                                                   \
      std::fprintf(stderr, "%s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                    \
    }                                                                \
  } while (0)

static SparseMlaParams sparse(int B, int T, int H, int D, int BM, int window, int topk, int max_seq, int ratio) {
  SparseMlaParams p;
  std::memset(&p, 0, sizeof(p));
  p.B = B;
  p.T = T;
  p.H = H;
  p.D = D;
  p.PAGE = 128;
  p.RATIO = ratio;
  p.MAX_SEQ = max_seq;
  p.ORI_BLOCKS = B * (max_seq / 128);
  p.CMP_BLOCKS = B * (max_seq / 128);
  p.WINDOW = window;
  p.TOPK = topk;
  p.S = window + (topk + 511) / 512 * 512;
  p.BM = BM;
  p.dtype = AFA_DTYPE_BF16;
  p.scale = 0.044f;
  return p;
}

static uint64_t round256(uint64_t n) { return (n + 255) / 256 * 256; }

int main() {
  // Workspace sizes: the plan (counts, then padded row lists) for whole-key
  // calls, plus split records for short streams; the formula in the header.
  const int batches[] = {1, 4, 16, 48, 64, 128, 1000};
  const int queries[] = {1, 6, 8192};
  const int heads[] = {32, 64, 128};
  const int dims[] = {128, 256, 512};
  const int tiles[] = {32, 64};
  const int topks[] = {1, 512, 2048, 8192};
  for (int b : batches)
    for (int q : queries)
      for (int h : heads)
        for (int d : dims)
          for (int bm : tiles)
            for (int topk : topks)
              for (int parts = 0; parts <= 8; parts += 4) {
                if ((int64_t)b * q > 65536 || h % bm != 0) continue;
                SparseMlaParams p = sparse(b, b * q, h, d, bm, 128, topk, 131072, 2);
                p.parts = parts;
                uint64_t bytes = 0;
                const int s = workspace_size_sparse_mla(&bytes, &p);
                EXPECT(s == 0);
                const uint64_t list_pad = (uint64_t)(128 + topk + 255) / 256 * 256;
                const uint64_t plan = round256(4ull * p.T) + 4ull * p.T * list_pad;
                EXPECT(bytes >= plan);
                if (parts == 1) EXPECT(bytes == round256(plan));
                uint64_t again = 0;
                EXPECT(workspace_size_sparse_mla(&again, &p) == 0 && again == bytes);  // a pure function of the sizes
              }
  {
    uint64_t bytes = 0;
    SparseMlaParams p = sparse(4, 16, 64, 512, 64, 128, 512, 4096, 2);
    EXPECT(workspace_size_sparse_mla(nullptr, &p) == AFA_E_NULL);
    EXPECT(workspace_size_sparse_mla(&bytes, nullptr) == AFA_E_NULL);
  }

  // Rejections, before any launch: sizes, dtype, ring, parts, overflow bounds.
  struct Bad {
    void (*edit)(SparseMlaParams&);
    int status;
  };
  const Bad bad[] = {
      {[](SparseMlaParams& p) { p.D = 384; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.BM = 16; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.H = 96; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.RATIO = 3; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.S = 100; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.scale = 0.0f; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.scale = -1.0f; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.dtype = 7; }, AFA_E_DTYPE},
      {[](SparseMlaParams& p) { p.ring = 5; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.parts = 9; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.parts = -1; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.B = 0; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.T = -5; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.MAX_SEQ = 100; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.WINDOW = 0; p.TOPK = 0; p.S = 0; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.TOPK = 9000; p.S = 128 + 9216; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.ORI_BLOCKS = 1 << 24; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.CMP_BLOCKS = 0; }, AFA_E_SHAPE},
      {[](SparseMlaParams& p) { p.T = 0x7fffffff; p.B = 1; }, AFA_E_SHAPE},
  };
  void* fake = reinterpret_cast<void*>(uintptr_t(256));
  const int32_t* ifake = reinterpret_cast<const int32_t*>(fake);
  for (const Bad& c : bad) {
    SparseMlaParams p = sparse(4, 16, 64, 512, 64, 128, 512, 4096, 2);
    c.edit(p);
    uint64_t bytes = 0;
    EXPECT(workspace_size_sparse_mla(&bytes, &p) == c.status);
    EXPECT(launch_sparse_mla(nullptr, fake, fake, fake, ifake, ifake, ifake, ifake, ifake, ifake, ifake, ifake,
                             reinterpret_cast<const float*>(fake), fake, fake, &p) == c.status);
    EXPECT(launch_sparse_mla_noalloc(nullptr, fake, fake, fake, ifake, ifake, ifake, ifake, ifake, ifake, ifake,
                                     ifake, reinterpret_cast<const float*>(fake), fake, &p) == c.status);
    EXPECT(launch_sparse_mla_planned(nullptr, fake, fake, fake, reinterpret_cast<const float*>(fake), fake, fake,
                                     &p) == c.status);
    EXPECT(launch_sparse_mla_plan(nullptr, ifake, ifake, ifake, ifake, ifake, ifake, ifake, ifake, fake, &p) ==
           c.status);
  }
  {
    SparseMlaParams p = sparse(4, 16, 64, 512, 64, 128, 512, 4096, 2);
    EXPECT(launch_sparse_mla(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                             nullptr, nullptr, nullptr, nullptr, nullptr, &p) == AFA_E_NULL);
    EXPECT(launch_sparse_mla(nullptr, fake, fake, fake, ifake, ifake, ifake, ifake, ifake, ifake, ifake, ifake,
                             reinterpret_cast<const float*>(fake), fake, fake, nullptr) == AFA_E_NULL);
    EXPECT(launch_sparse_mla_planned(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &p) ==
           AFA_E_NULL);
    p.debug_rows = const_cast<int32_t*>(ifake);
    EXPECT(launch_sparse_mla_planned(nullptr, fake, fake, fake, reinterpret_cast<const float*>(fake), fake, fake,
                                     &p) == AFA_E_SHAPE);
  }

  // Top-k rejections.
  {
    SparseTopkParams p;
    std::memset(&p, 0, sizeof(p));
    p.B = 1;
    p.T = 4;
    p.TOPK = 512;
    p.RATIO = 2;
    p.C = 1024;
    EXPECT(launch_sparse_topk_indices(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &p) == AFA_E_NULL);
    EXPECT(launch_sparse_topk_indices(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) == AFA_E_NULL);
    const float* f = reinterpret_cast<const float*>(fake);
    int32_t* o = reinterpret_cast<int32_t*>(fake);
    SparseTopkParams q = p;
    q.C = int64_t(1) << 31;
    EXPECT(launch_sparse_topk_indices(nullptr, f, ifake, ifake, ifake, o, &q) == AFA_E_SHAPE);
    q = p;
    q.RATIO = 3;
    EXPECT(launch_sparse_topk_indices(nullptr, f, ifake, ifake, ifake, o, &q) == AFA_E_SHAPE);
    q = p;
    q.TOPK = 0;
    EXPECT(launch_sparse_topk_indices(nullptr, f, ifake, ifake, ifake, o, &q) == AFA_E_SHAPE);
  }

  // Dense kernels: sizes and rejections.
  {
    FaParams fa;
    std::memset(&fa, 0, sizeof(fa));
    fa.B = 1;
    fa.HQ = 8;
    fa.HKV = 8;
    fa.D = 128;
    fa.dtype = AFA_DTYPE_F16;
    fa.scale = 0.088f;
    uint64_t bytes = 1;
    EXPECT(workspace_size_attention_target(&bytes, 8, 8, &fa) == 0 && bytes == 0);
    EXPECT(workspace_size_simple_attention(&bytes, 256, 4) == 0 && bytes == 0);
    EXPECT(workspace_size_simple_attention(nullptr, 64, 1) == AFA_E_NULL);
    EXPECT(launch_attention_target(nullptr, fake, fake, fake, fake, nullptr, 0, 8, &fa) == AFA_E_SHAPE);
    fa.HKV = 3;
    EXPECT(launch_attention_target(nullptr, fake, fake, fake, fake, nullptr, 8, 8, &fa) == AFA_E_SHAPE);
    EXPECT(launch_simple_attention(nullptr, fake, fake, fake, fake, nullptr, 100, 1) == AFA_E_SHAPE);
  }

  // Metadata and config queries: well-formed, stable strings and vectors.
  {
    const char* metas[] = {kernel_metadata_sparse_mla(), kernel_metadata_attention_target(),
                           kernel_metadata_simple_attention()};
    for (const char* m : metas) {
      EXPECT(m != nullptr && std::strlen(m) > 16 && m[0] == '{' && m[std::strlen(m) - 1] == '}');
    }
    EXPECT(std::strstr(metas[0], "\"ring\"") != nullptr);
    int64_t cfg[5];
    EXPECT(kernel_config_sparse_mla(cfg) == 0 && cfg[0] == 13 && cfg[2] == 1);
    EXPECT(kernel_config_attention_target(cfg) == 0);
    EXPECT(kernel_config_simple_attention(cfg) == 0);
    EXPECT(kernel_config_sparse_mla(nullptr) == AFA_E_NULL);
    const char* version = ascendflow_amd_version();
    EXPECT(version != nullptr && std::strstr(version, "gfx950") != nullptr);
  }

  if (failures) {
    std::fprintf(stderr, "%d host check(s) failed\n", failures);
    return 1;
  }
  std::printf("host ABI checks passed\n");
  return 0;
}
