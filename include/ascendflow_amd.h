/*
 * ascendflow_amd C ABI: MI355X (gfx950) sparse-MLA and flash-attention launchers.
 *
 * Drop-in counterparts of the launchers the reference's back end emits for its
 * three attention operators (src/backend/structured.py:573-649):
 *   int launch_<k>(void* stream, void* arg_<tensor>..., [void* workspace], [int64 sizes]);
 *   int kernel_config_<k>(int64_t cfg[5]);
 *   const char* kernel_metadata_<k>(void);
 *   int workspace_size_<k>(uint64_t* bytes, ...);   (src/backend/workspace.py:100-130)
 *
 * The reference specialises every size as a DSL constexpr; here the sizes are
 * runtime fields of a small parameter struct passed by pointer, because the
 * drop-in surface is the Python entry signature, not the Ascend binary.
 *
 * Conventions (all entry points):
 *  - every tensor argument is a device pointer to contiguous row-major memory;
 *    the caller allocates all tensors, outputs included, and keeps them
 *    pairwise disjoint (docs/guide/runtime.md:86-89 in the reference);
 *  - launches are asynchronous on `stream` (a hipStream_t, NULL = default);
 *  - return value: 0 on success, a negative AFA_E* code for a rejected
 *    configuration, or a positive hipError_t if the launch itself failed.
 *    Nothing is retried (src/runtime/kernel.py:59-63).
 */
#ifndef ASCENDFLOW_AMD_H
#define ASCENDFLOW_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  AFA_OK = 0,
  AFA_E_NULL = -1,        /* a required pointer is NULL */
  AFA_E_SHAPE = -2,       /* unsupported or inconsistent size */
  AFA_E_DTYPE = -3,       /* unsupported storage dtype */
  AFA_E_WORKSPACE = -4,   /* workspace missing or too small */
};

enum { AFA_DTYPE_BF16 = 0, AFA_DTYPE_F16 = 1 };

/* Sizes and policy of one sparse_mla call
 * (examples/sparse_attention/attention.py:225-245). */
typedef struct SparseMlaParams {
  int32_t B, T, H, D;
  int32_t PAGE, RATIO, MAX_SEQ;
  int32_t ORI_BLOCKS, CMP_BLOCKS;
  int32_t WINDOW, TOPK, S, BM;
  int32_t dtype;            /* AFA_DTYPE_* of q, caches and attention_out */
  float scale;              /* SCALE, > 0 */
  /* Parts each (token, BM-head tile) key is split into, with a workspace: 0 =
   * automatic (after at most one full round of keys over 256 compute units,
   * the keys of the incomplete last round, into the number of parts a cost
   * model of the GPU finds cheapest, if any: decode with few requests), 1 =
   * never, 2..8 = every key. Parts run on different workgroups and store their
   * output normalised by their own denominator, with their running max and
   * denominator; a merge kernel combines them in part order, so results are
   * deterministic for a given value. No counterpart in the reference, whose
   * sizes are compile-time constants. */
  int32_t parts;
  /* KV ring of the persistent kernel (the plan path): 0 = automatic, 3 or 4
   * tiles of 32 rows. Three tiles keep one chunk in flight, four keep two.
   * Automatic takes four when ori_kv and cmp_kv together exceed MI355X's
   * 256 MiB Infinity Cache (rows then mostly come from HBM), else three; four
   * tiles are used only where the row-list ring fits next to them in LDS
   * (otherwise three). Results are bit-identical either way. No counterpart
   * in the reference. */
  int32_t ring;
  /* Optional debug image of the row selection, NULL normally: int32 [T, S, 2].
   * Entry r < n of token t is the r-th row of the compacted row list the
   * attention kernel streams for t (the LDS list it attends over, copied out
   * after it is built), as (cache, physical_row), cache 0 = ori_kv,
   * 1 = cmp_kv, in slot order (window positions, then compressed ranks,
   * duplicates kept); entries from n on are (-1, -1). A call with it set
   * resolves rows inside the attention kernel and splits no key. The
   * per-slot layout of the reference's gather workspace is
   * launch_sparse_mla_gather's. */
  int32_t* debug_rows;
  /* Optional f32 [T, H] output, NULL normally: the natural-log softmax
   * normaliser ln(sum_j e^(s_j) + e^sink[h]) of each (token, head), s_j =
   * SCALE * q.k_j over the selected rows (the sink alone for an empty
   * selection), i.e. the denominator of attention_out. The counterpart of the
   * softmax_lse output of the vendor operator the reference benchmarks against
   * (aclnnSparseFlashMla, benchmarks/references/sparse_mla_aclnn.py:100-130),
   * which the DSL kernel itself does not produce. */
  float* softmax_lse;
} SparseMlaParams;

/* Sparse MLA forward: examples/sparse_attention/attention.py:210-525.
 * Tensor order is the reference entry order (attention.py:211-224):
 *   q [T,H,D], ori_kv [ORI_BLOCKS,PAGE,1,D], cmp_kv [CMP_BLOCKS,PAGE/RATIO,1,D],
 *   cmp_sparse_indices i32 [T,1,TOPK], ori_block_table i32 [B,MAX_SEQ/PAGE],
 *   cmp_block_table i32 [B,MAX_SEQ/PAGE], cu_seqlens_q i32 [B+1],
 *   seqused_ori_kv i32 [B], seqused_cmp_kv i32 [B], cmp_residual_kv i32 [B],
 *   ori_topk_length i32 [T,1], sinks f32 [H], attention_out [T,H,D] (written).
 * `workspace`: NULL, or at least workspace_size_sparse_mla() bytes of device
 * memory that the call may overwrite. With a workspace and at least two work
 * items (token x BM-head tile) per compute unit, a plan kernel first writes
 * every token's selected-row list into it and a persistent attention kernel
 * streams the items of each compute unit over those lists. The plan is:
 * int32 counts [T] at byte 0 (selected rows per token), then, from byte
 * round_up(4 T, 256), uint32 lists [T][round_up(WINDOW + TOPK, 256)] of
 * tagged rows (bit 31 set: cmp_kv row, else ori_kv row; physical row in the
 * low bits) in slot order, padded with the token's first row to a multiple of
 * 32 entries (32 entries of ori_kv row 0 for an empty selection); otherwise (or with
 * params->debug_rows set) one workgroup per item (or per part of a split key,
 * params->parts, whose records a merge kernel then combines in the workspace)
 * resolves its rows itself. With one part, results are bit-identical either
 * way; split keys differ only in FP32 summation order. */
int launch_sparse_mla(void* stream, const void* q, const void* ori_kv, const void* cmp_kv,
                      const int32_t* cmp_sparse_indices, const int32_t* ori_block_table,
                      const int32_t* cmp_block_table, const int32_t* cu_seqlens_q,
                      const int32_t* seqused_ori_kv, const int32_t* seqused_cmp_kv,
                      const int32_t* cmp_residual_kv, const int32_t* ori_topk_length,
                      const float* sinks, void* attention_out, void* workspace,
                      const SparseMlaParams* params);

/* Allocation-free variant of launch_sparse_mla, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference, whose
 * runtime owns a workspace arena per stream binding (src/runtime/kernel.py:39-49).
 * Same arguments without `workspace`: the call's workspace (row-list plan and
 * split records, workspace_size_sparse_mla bytes) lives in a static device
 * array of 32 MiB per GPU (AFA_SCRATCH_BYTES), resolved once per device; it
 * allocates nothing. Returns AFA_E_WORKSPACE, before any launch, when the
 * call's workspace exceeds it (e.g. a 32K-token prefill: 100 MiB). Results are
 * bit-identical to launch_sparse_mla with a workspace. All calls on one GPU
 * share the array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller. */
#define AFA_SCRATCH_BYTES (32u << 20)
int launch_sparse_mla_noalloc(void* stream, const void* q, const void* ori_kv, const void* cmp_kv,
                              const int32_t* cmp_sparse_indices, const int32_t* ori_block_table,
                              const int32_t* cmp_block_table, const int32_t* cu_seqlens_q,
                              const int32_t* seqused_ori_kv, const int32_t* seqused_cmp_kv,
                              const int32_t* cmp_residual_kv, const int32_t* ori_topk_length,
                              const float* sinks, void* attention_out, const SparseMlaParams* params);

/* Gather image of the sparse selection, the layout of the reference's gather
 * workspace and of its gather oracle (benchmarks/attention/sparse_reference.py:174-181,
 * examples/sparse_attention/gather.py:86-131, window slots from gather.py:38-60):
 *   kv_out [T,S,D] (dtype of the caches; unused slots zero),
 *   bias_out f32 [T,S] (0 selected, -inf unused).
 * Uses the fused kernel's own slot resolution and row copy. */
int launch_sparse_mla_gather(void* stream, const void* ori_kv, const void* cmp_kv,
                             const int32_t* cmp_sparse_indices, const int32_t* ori_block_table,
                             const int32_t* cmp_block_table, const int32_t* cu_seqlens_q,
                             const int32_t* seqused_ori_kv, const int32_t* seqused_cmp_kv,
                             const int32_t* cmp_residual_kv, const int32_t* ori_topk_length,
                             void* kv_out, float* bias_out, const SparseMlaParams* params);

/* Flash attention (BNSD): examples/flash_attention/attention.py:243-417.
 *   Q [B,HQ,Sq,D], K/V [B,HKV,Sk,D], O [B,HQ,Sq,D] (written).
 * The reference launcher is (stream, Q, K, V, O, workspace, Sq, Sk). */
typedef struct FaParams {
  int32_t B, HQ, HKV, D;
  int32_t dtype;   /* AFA_DTYPE_* */
  int32_t causal;  /* top-left j <= i masking (attention.py:96-110) */
  float scale;
  int32_t reserved;
} FaParams;

int launch_attention_target(void* stream, const void* Q, const void* K, const void* V, void* O,
                            void* workspace, int64_t Sq, int64_t Sk, const FaParams* params);

/* Teaching attention: examples/flash_attention/simple.py:60-141.
 *   Q [H,S,128] f16, K/V [H,128,128] f16, O [H,S,128] f16 (written);
 * softmax(QK^T / sqrt(128)) normalised before the f16 cast of P. */
int launch_simple_attention(void* stream, const void* Q, const void* K, const void* V, void* O,
                            void* workspace, int64_t S, int64_t H);

/* kernel_config_<k>: cfg[5] = {tensors, runtime parameters, has_workspace,
 * compute units, SIMDs per CU} (src/backend/structured.py:619-637). */
int kernel_config_sparse_mla(int64_t cfg[5]);
int kernel_config_attention_target(int64_t cfg[5]);
int kernel_config_simple_attention(int64_t cfg[5]);

/* kernel_metadata_<k>: versioned JSON naming tensors, dtypes, shapes and
 * access modes (src/backend/abi.py:19-59). Static storage. */
const char* kernel_metadata_sparse_mla(void);
const char* kernel_metadata_attention_target(void);
const char* kernel_metadata_simple_attention(void);

/* workspace_size_<k>: bytes of the optional workspace (sparse_mla: the row-list
 * plan, T * 4 rounded up to 256 plus T * round_up(WINDOW + TOPK, 256) * 4, and
 * with K (token, BM-head tile) keys split into P parts, rounded up to 256,
 * plus K * P * (2 * BM * D + BM * BM / 2) bytes of partial results; 0 for the
 * two dense kernels); returns -1 on a NULL pointer and the
 * launcher's status for invalid sparse parameters (src/backend/workspace.py:100-130). */
int workspace_size_sparse_mla(uint64_t* bytes, const SparseMlaParams* params);
int workspace_size_attention_target(uint64_t* bytes, int64_t Sq, int64_t Sk,
                                    const FaParams* params);
int workspace_size_simple_attention(uint64_t* bytes, int64_t S, int64_t H);

/* The row-list plan alone: writes the plan that launch_sparse_mla's plan
 * kernel writes into its workspace (layout above) for every token, nothing
 * else. The counterpart of the vendor operator's metadata-preparation stage
 * (docs/operators/sparse-mla.md:10-14 in the reference); used to read the
 * selection back and to drive launch_gather_probe. `workspace` needs
 * round_up(4 T, 256) + 4 T round_up(WINDOW + TOPK, 256) bytes. */
int launch_sparse_mla_plan(void* stream, const int32_t* cmp_sparse_indices, const int32_t* ori_block_table,
                           const int32_t* cmp_block_table, const int32_t* cu_seqlens_q,
                           const int32_t* seqused_ori_kv, const int32_t* seqused_cmp_kv,
                           const int32_t* cmp_residual_kv, const int32_t* ori_topk_length, void* workspace,
                           const SparseMlaParams* params);

/* The attention over a plan alone: the persistent kernel of launch_sparse_mla
 * (one workgroup per compute unit streaming its tokens' row lists, KV ring
 * per params->ring) over the plan that launch_sparse_mla_plan wrote into
 * `workspace` for the same metadata and params. The two calls together give
 * launch_sparse_mla's output (and softmax_lse) bit for bit; the persistent
 * kernel runs here whatever T is, and no key is split. Lets a caller run the
 * plan ahead on another stream or reuse one plan for several calls over the
 * same selection. The plan must come from launch_sparse_mla_plan with the
 * same metadata and params (whether a launch_sparse_mla call wrote one depends
 * on the device and the split, so its workspace is not a plan to rely on).
 * Counts and row ids read from `workspace` are clamped to the list capacity
 * and to ori_kv / cmp_kv, so a workspace holding anything else gives a wrong
 * output but no access outside the caches. No counterpart in the
 * reference, whose operator is one kernel. Returns AFA_E_SHAPE when
 * params->debug_rows is set (the plan path writes no debug image) or no KV
 * ring fits next to the row lists (at D = 512, WINDOW + TOPK above 3328). */
int launch_sparse_mla_planned(void* stream, const void* q, const void* ori_kv, const void* cmp_kv,
                              const float* sinks, void* attention_out, const void* workspace,
                              const SparseMlaParams* params);

/* Gather probe (measurement only; the counterpart of the reference's gather
 * micro-benchmark, benchmarks/attention/gather_dma.py): streams the 1 KiB rows
 * listed in a plan (D = 512, one item per token: BM = H) from ori_kv/cmp_kv
 * through LDS as the attention kernels do, with `depth` (1, 2, 4, 6 or 8)
 * 16-row chunks in flight per workgroup and no compute, on `grid`
 * workgroups: items interleaved (balanced = 0) or an equal share of the flat
 * chunk stream each (balanced = 1, every item taken as long as item 0). Each
 * workgroup takes at most 4 items. sums [grid][16]: per thread, the sum of the
 * first dword of every row it checked (all rows streamed, mod 2^32). */
int launch_gather_probe(void* stream, const void* ori_kv, const void* cmp_kv, const void* workspace,
                        const SparseMlaParams* params, int32_t grid, int32_t depth, int32_t balanced,
                        uint32_t* sums);

/* Top-k index selection: the producer of cmp_sparse_indices, which the
 * reference takes as an input and leaves to the caller's indexer
 * (docs/operators/sparse-mla.md:8,266 in the reference). scores [T][C] f32: one
 * index score per (token, compressed position). For token t of request b
 * (cu_seqlens_q), with n queries in b, offset j and cutoff = max(0,
 * seqused_cmp_kv[b] RATIO + cmp_residual_kv[b] - n + j + 1) / RATIO (the
 * causal bound of the sparse contract, docs/operators/sparse-mla.md:41-51),
 * writes into cmp_sparse_indices [T][1][TOPK] the min(TOPK, seqused_cmp_kv[b],
 * cutoff, C) positions p < min(cutoff, C) of largest score, ascending, then
 * -1 (the input contract of docs/operators/sparse-mla.md:79). Ties go to the
 * lower position; -0 equals +0; NaN ranks above +inf. Returns AFA_E_SHAPE for
 * B, T, TOPK or C <= 0, C >= 2^31 or RATIO not 1 or 2, AFA_E_NULL for a NULL
 * pointer, before any launch. One launch; no workspace. */
typedef struct SparseTopkParams {
  int32_t B;      /* requests */
  int32_t T;      /* query tokens */
  int32_t TOPK;   /* selected positions per token (row length of the output) */
  int32_t RATIO;  /* compression ratio, 1 or 2 */
  int64_t C;      /* score columns per token (row stride of scores), < 2^31 */
} SparseTopkParams;

int launch_sparse_topk_indices(void* stream, const float* scores, const int32_t* cu_seqlens_q,
                               const int32_t* seqused_cmp_kv, const int32_t* cmp_residual_kv,
                               int32_t* cmp_sparse_indices, const SparseTopkParams* params);

/* Measurement helpers (no reference kernel; the reference sweeps a >= 4x L2
 * buffer before each timed launch, benchmarks/cache.py:13-92 and
 * benchmarks/cache_sweep.py:15-32). Reads `bytes` of `buffer` through the
 * caches (cached 16-byte loads, nothing written back for a zero-filled
 * buffer) so that the next launch starts cold. */
int launch_cache_flush(void* stream, void* buffer, uint64_t bytes);

/* Measurement helper (no reference kernel): runs `spins` dependent FMAs in
 * every thread of 1024 workgroups of 256 (every SIMD busy) and writes, from
 * workgroup 0, out[0..1] = the shader-cycle counter before and after and
 * out[2..3] = the 100 MHz real-time counter before and after (out has 5
 * entries): the shader clock is 100 MHz x (out[1] - out[0]) / (out[3] - out[2]). */
int launch_clock_probe(void* stream, uint64_t* out, int32_t spins);

/* Library version string. */
const char* ascendflow_amd_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ASCENDFLOW_AMD_H */
