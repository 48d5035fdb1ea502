/*
 * qraf_hip.h -- C ABI of the MI355X (gfx950) QRAF decode hot path.
 *
 * A drop-in for the dispatch layer of simonpierreboucher02/qraf
 * (include/nn/backend.h, src/nn/backend.cpp) and for the per-token engine
 * below it (src/nn/transformer.cpp, src/nn/attention.cpp).  Plain C types
 * only: pointers, sizes, dtype codes of include/core/types.h:27-39
 * (F32 = 0, F16 = 1, Q8_0 = 10, Q4_0 = 20) and block sizes from
 * QuantScheme.block_size (include/qraf/format.h:88-97).
 *
 * Every function returns QRAF_HIP_OK (0) or a negative QRAF_HIP_ERR_* code;
 * qraf_hip_last_error() describes the calling thread's last failure.  Where
 * the reference silently zero-fills (unknown dtype in dispatch_matvec_q,
 * backend.cpp:195-198) this library returns QRAF_HIP_ERR_DTYPE instead; the
 * C++ shim in INTEGRATION.md turns nonzero codes into qraf::QrafError.
 *
 * Pointer kinds: functions named *_dev take device pointers and a stream
 * (hipStream_t passed as void*, NULL = the library's default stream) and
 * are stream-ordered; every other compute function takes host pointers and
 * returns after its result is in host memory.
 */
#ifndef QRAF_HIP_H
#define QRAF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QRAF_HIP_OK 0
#define QRAF_HIP_ERR_INVALID (-1) /* bad argument or shape            */
#define QRAF_HIP_ERR_DTYPE (-2)   /* unsupported dtype / block size    */
#define QRAF_HIP_ERR_HIP (-3)     /* HIP runtime failure               */
#define QRAF_HIP_ERR_NOMEM (-4)   /* device or page-pool exhaustion    */
#define QRAF_HIP_ERR_STATE (-5)   /* call not valid in the current state */
#define QRAF_HIP_ERR_FORMAT (-6)  /* malformed QRAF file                */

#define QRAF_DTYPE_F32 0u
#define QRAF_DTYPE_F16 1u
#define QRAF_DTYPE_Q8_0 10u
#define QRAF_DTYPE_Q4_0 20u
#define QRAF_DTYPE_I8 102u /* KV pages only: the QuantizedKVCache scheme, kv_cache_quant.h:61-128 */

/* ------------------------------------------------------------ runtime */

/* Last error of the calling thread ("" if none). */
const char* qraf_hip_last_error(void);
/* Select the device and create the library's default stream.  Replaces
 * backend_init() (backend.cpp:18-50) for the HIP backend; idempotent. */
int qraf_hip_init(int device);
int qraf_hip_device_count(int* count);
/* Build information: "gfx950 <compiler version>". */
const char* qraf_hip_version(void);

/* Device memory, streams, events and graphs, so callers need no HIP headers. */
int qraf_hip_malloc(void** dev_ptr, uint64_t bytes);
int qraf_hip_free(void* dev_ptr);
int qraf_hip_memcpy_h2d(void* dst_dev, const void* src_host, uint64_t bytes);
int qraf_hip_memcpy_d2h(void* dst_host, const void* src_dev, uint64_t bytes);
int qraf_hip_memcpy_d2d(void* dst_dev, const void* src_dev, uint64_t bytes, void* stream);
int qraf_hip_memset(void* dev_ptr, int value, uint64_t bytes);
/* Streaming read of `bytes` (a positive multiple of 16, 16-byte aligned) in
 * the device's best plain-read launch shape: the HBM ceiling a memory-bound
 * kernel moving the same bytes is measured against.  Writes partial sums of
 * the data to `out` (qraf_hip_read_probe_out_bytes bytes).  No counterpart in
 * the reference (a measurement aid). */
int qraf_hip_read_probe_dev(const void* dev_ptr, uint64_t bytes, float* out, void* stream);
uint64_t qraf_hip_read_probe_out_bytes(void);
/* One launch of an empty kernel over `workgroups` (1..65536) 64-thread
 * workgroups on `stream`: the fixed cost every launch pays, measured the way
 * a step's kernels run (back to back in a graph).  No counterpart in the
 * reference: a measurement entry point. */
int qraf_hip_launch_floor_dev(int32_t workgroups, void* stream);
int qraf_hip_stream_create(void** stream);
int qraf_hip_stream_destroy(void* stream);
int qraf_hip_stream_synchronize(void* stream);
int qraf_hip_device_synchronize(void);
int qraf_hip_event_create(void** event);
int qraf_hip_event_destroy(void* event);
int qraf_hip_event_record(void* event, void* stream);
int qraf_hip_event_elapsed_ms(void* start, void* stop, float* ms);
/* Capture stream-ordered library calls made on `stream` into a graph. */
int qraf_hip_graph_begin(void* stream);
int qraf_hip_graph_end(void* stream, void** graph_exec);
int qraf_hip_graph_launch(void* graph_exec, void* stream);
int qraf_hip_graph_destroy(void* graph_exec);

/* ------------------------------------------------ op level (backend.h) */

/* Weight residency for the op-level calls: a host weight buffer registered
 * here is copied to HBM once and every later op-level call that passes the
 * same host pointer reads the HBM copy.  Mirrors how the reference keeps
 * weights as immutable mmap views (loader.cpp:236-258). */
int qraf_hip_register_weights(const void* host_ptr, uint64_t bytes);
int qraf_hip_unregister_weights(const void* host_ptr);

/* dispatch_matvec_q (backend.h:31-34, backend.cpp:131-199):
 * y[i] = dot(row_i(w), x) for i < out_dim; w in the reference's Q8_0/Q4_0
 * block layout with `block_size` (0 means 32, as backend.cpp:135).
 * w_size may be 0 (unchecked, as the reference) or the buffer size. */
int qraf_hip_matvec_q(const void* w, uint64_t w_size, uint32_t dtype, uint32_t block_size,
                      uint32_t out_dim, uint32_t in_dim, const float* x, float* y);
/* dispatch_matvec_opt (backend.h:27-28, backend.cpp:62-105). */
int qraf_hip_matvec_f32(const float* W, const float* x, float* y, uint32_t out_dim, uint32_t in_dim);
/* dispatch_dot_f32 (backend.h:37, backend.cpp:109-127). */
int qraf_hip_dot_f32(const float* a, const float* b, int n, float* result);
/* dispatch_rms_norm / softmax / silu / add / mul / scale
 * (backend.h:40-45, backend.cpp:203-320). */
int qraf_hip_rms_norm(float* x, const float* weight, int size, float eps);
int qraf_hip_softmax(float* x, int size);
int qraf_hip_silu(float* x, int size);
int qraf_hip_add(float* x, const float* y, int size);
int qraf_hip_mul(float* x, const float* y, int size);
int qraf_hip_scale(float* x, float s, int size);

/* --------------------------------------------------- device level */

/* Device-pointer form of qraf_hip_matvec_q; stream-ordered. */
int qraf_hip_matvec_q_dev(const void* w, uint32_t dtype, uint32_t block_size, uint32_t out_dim,
                          uint32_t in_dim, const float* x, float* y, void* stream);
int qraf_hip_matvec_f32_dev(const float* W, const float* x, float* y, uint32_t out_dim,
                            uint32_t in_dim, void* stream);
/* dispatch_matvec_q (backend.h:31-34, backend.cpp:131-199) applied to each of
 * `batch` activation rows at once: y[b][out_dim] = W x[b] for b < batch,
 * x [batch][in_dim] and y [batch][out_dim] on the device, stream-ordered.
 * Every weight unit is read once for all rows, each row's sum running the
 * batch-1 persistent kernel's arithmetic.  Q8_0 / Q4_0 with block size 32;
 * batch 1..16; in_dim a multiple of 32 (of 64 for Q4_0) such that the
 * batch rounded up to 2, 4, 8 or 16, times in_dim, fits the kernel's LDS
 * staging (144 KB: 32,768 elements for Q8_0, 31,040 for Q4_0); anything
 * else is an error (the batched GEMM takes larger batches).  The engine runs steps of 2-8 rows this way where every
 * projection fits. */
int qraf_hip_matvec_q_batch_dev(const void* w, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                                const float* x, int32_t batch, float* y, void* stream);
/* Tuning of the batch-1 kernel (process-wide): kernel 0 = automatic,
 * 1 = one-shot, 2 = persistent streaming, 3 / 4 = ring with workgroups of
 * 8 / 4 waves (the automatic choice is 3 when K % 32 == 0, x is 16-byte
 * aligned and x fits the ring's staging); rows per wave 0 (automatic), 1, 2,
 * 4 or 8 (the ring kernel takes 1 or 2); workgroups per CU for the
 * persistent and ring kernels (0 = automatic). */
int qraf_hip_set_matvec_tuning(int kernel, int rows, int wgs_per_cu);

/* quantize_q8_0 / quantize_q4_0 (quantize.cpp:105-183) on the device, block
 * size 32, bit-exact with the reference: `count` fp32 values -> `dst` in the
 * reference block layout (ceil(count/32) blocks). */
int qraf_hip_quantize_dev(const float* src, uint64_t count, uint32_t dtype, void* dst, void* stream);
/* Synthetic weights for benchmarks and tests (the role of
 * tools/dummy_model.cpp:12-17): `count` values N(0, stddev) from the
 * repository's counter-based generator (seed, stream_id), written as F32 or
 * quantized to Q8_0/Q4_0 as by qraf_hip_quantize_dev.  stream_id is
 * conventionally qraf_hip_name_hash(tensor name). */
int qraf_hip_gen_weights_dev(void* dst, uint32_t dtype, uint64_t count, uint64_t seed, uint64_t stream_id,
                             float stddev, void* stream);
/* FNV-1a of a tensor name (format.h:136-147); returns the hash itself. */
uint64_t qraf_hip_name_hash(const char* name);

/* ------------------------------------------- ragged paged decode attention */

/* Workspace bytes for qraf_hip_paged_attention_dev (partials of contexts
 * split across workgroups); no initialisation needed.  Calls sharing one
 * must not overlap. */
uint64_t qraf_hip_attention_workspace_bytes(int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads,
                                            int32_t head_dim, int32_t max_ctx);
/* The score / softmax / weighted-sum loops of attention_forward
 * (attention.cpp:122-150) for a ragged batch of n_seqs sequences that each
 * attend with one query token:
 *   q        [n_seqs][n_heads][head_dim] f32, RoPE already applied
 *   k_cache  [num_pages][n_kv_heads][page_size][head_dim], F32 or F16
 *   v_cache  F32: [num_pages][n_kv_heads][page_size][head_dim]
 *            F16: [num_pages][n_kv_heads][head_dim][page_size] (dimension-major
 *            in a page, the layout qraf_hip_rope_append_dev writes)
 *   I8 (both caches): [num_pages][n_kv_heads] blocks of page_size*(head_dim+4)
 *            bytes; K block = int8 [page_size][head_dim] then f32 scale
 *            [page_size], V block = int8 [head_dim][page_size] then f32 scale
 *            [page_size]; a score is (sum q_k[d]*query[d]) * k_scale * scale
 *            (dot_with_key, kv_cache_quant.h:118-128), a value q_v[d]*v_scale
 *            (dequant_value, :108-116)
 *   page_table [n_seqs][max_pages_per_seq] physical page of logical page j
 *   ctx_lens [n_seqs] positions attended (1 <= ctx <= max_ctx), on the device
 *   out      [n_seqs][n_heads][head_dim] f32
 * Query head h reads KV head h / (n_heads / n_kv_heads) (attention.cpp:127);
 * scale is 1/sqrt(head_dim) in the reference (attention.cpp:122).
 * head_dim 64 or 128 with n_heads / n_kv_heads in {1,2,3,4,6,8,12,16}, or
 * head_dim 16 or 32 with n_heads / n_kv_heads in {1,2,4,8}.  F32 and F16
 * pages with head_dim 64/128, at most 16 query heads per KV head and a
 * power-of-two page_size >= 4 run on the matrix cores (F32 pages in fp32
 * arithmetic throughout); I8 pages need that shape (QRAF_HIP_ERR_INVALID
 * otherwise) and always do.  Page
 * contents at positions >= ctx are never used (NaN there is harmless). */
/* Work decomposition of the matrix-core attention (process-wide):
 * 1 = one workgroup per (sequence, 256-position chunk), 2 = balanced split
 * of the batch's 64-position tiles over the resident workgroups,
 * 0 = automatic (default: the split when n_seqs * ceil(max_ctx / 256)
 * exceeds 1024, else the chunk grid), 3 = the plain fp32 VALU kernel for F32
 * and F16 pages (I8 pages: automatic).  Results agree within the attention
 * tolerance, not bit for bit. */
int qraf_hip_set_attention_tuning(int32_t form);
int qraf_hip_paged_attention_dev(const float* q, const void* k_cache, const void* v_cache, uint32_t kv_dtype,
                                 const int32_t* page_table, int32_t max_pages_per_seq, const int32_t* ctx_lens,
                                 int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                 int32_t page_size, float scale, int32_t max_ctx, float* out, void* workspace,
                                 uint64_t workspace_bytes, void* stream);
/* qraf_hip_paged_attention_dev without a workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The workspace is a file-scope device array of
 * qraf_hip_attention_noalloc_max_bytes() bytes (32 MiB) per GPU, resolved by
 * qraf_hip_init (QRAF_HIP_ERR_STATE if that was not called on the current
 * device); a shape whose qraf_hip_attention_workspace_bytes exceeds it is
 * refused with QRAF_HIP_ERR_INVALID.  The call allocates nothing.  Every call
 * on one GPU uses the same array: calls that overlap on one GPU (other
 * streams, other threads) race. */
int qraf_hip_paged_attention_noalloc_dev(const float* q, const void* k_cache, const void* v_cache, uint32_t kv_dtype,
                                         const int32_t* page_table, int32_t max_pages_per_seq, const int32_t* ctx_lens,
                                         int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                         int32_t page_size, float scale, int32_t max_ctx, float* out, void* stream);
uint64_t qraf_hip_attention_noalloc_max_bytes(void);
/* RoPE angle table, RopeCache::init (ops.cpp:179-193) computed on the host
 * with the host libm: table[pos*head_dim + i] = cos(pos*f_i),
 * table[pos*head_dim + i + 1] = sin(pos*f_i), f_i = 1/powf(theta, i/head_dim)
 * for even i < head_dim; `table` holds max_pos*head_dim floats. */
int qraf_hip_rope_table_host(int32_t max_pos, int32_t head_dim, float rope_theta, float* table);
/* Bias add + interleaved-pair RoPE + cache store for one new token per
 * sequence (attention.cpp:100-119, ops.cpp:158-177): qkv [n_seqs][(H+2Hkv)*hd]
 * rows of the fused q|k|v projection, bias the matching F32 vector or NULL,
 * rope_table a device copy of the qraf_hip_rope_table_host table covering
 * every position; writes rotated q to q_out [n_seqs][H*hd] and rotated k, v at
 * positions[s] into the paged cache.  I8 pages: k and v quantized per KV head
 * as QuantizedKVCache::store (kv_cache_quant.h:61-95), bytes and scales
 * bit-identical to it; head_dim <= 128, page_size % 4 == 0 (attention on
 * them also needs a power of two). */
int qraf_hip_rope_append_dev(const float* qkv, const float* bias, int32_t n_seqs, int32_t n_heads,
                             int32_t n_kv_heads, int32_t head_dim, const int32_t* positions, const float* rope_table,
                             float* q_out, void* k_cache, void* v_cache, uint32_t kv_dtype, const int32_t* page_table,
                             int32_t max_pages_per_seq, int32_t page_size, void* stream);

/* ------------------------------------------------- batched quantized GEMM */

/* Split fp32 activations into two 16-bit planes, the operand form of
 * qraf_hip_qgemm_dev: x_hi = bf16 of x, x_lo = fp16 of x - x_hi (clamped to
 * +-65504), both round-to-nearest-even; x = hi + lo + r with
 * |r| <= 2^-20 |x| + 2^-25 for |x| < 2^24 (|r| <= 2^-8 |x| beyond).  rows x
 * cols elements, row-major. */
int qraf_hip_split_bf16_dev(const float* x, uint16_t* x_hi, uint16_t* x_lo, int32_t rows, int32_t cols,
                            void* stream);
/* Tuning of the batched GEMM for batches over 32 rows: waves 4 or 8 per
 * workgroup (128 or 256 weight rows), splits > 0 forces the split count,
 * pipe 1 / -1 forces the pipelined tiled kernel on / off, batch_chunk 16,
 * 32, 64 or 128 caps the batch rows one workgroup covers; 0 restores the
 * automatic choice.  Affects the workspace queries too.  No counterpart in
 * the reference (a performance knob). */
int qraf_hip_set_qgemm_tuning(int waves, int splits, int pipe, int batch_chunk);
/* Work schedule of the pipelined GEMM (batches over 32 rows, tile-major
 * weights): mode 1 = stream-K (each resident workgroup takes an equal share
 * of the (weight tile, quant block) pairs, at least min_blocks blocks (0:
 * 16), crossing tile boundaries; a tile's segments are summed in segment
 * order, so results stay deterministic), 2 and 0 (the default) = the
 * uniform split-K grid, which measured faster at the continuous-batch
 * shapes (shares of 11-21 blocks pay a pipeline prologue per segment).  A
 * forced split count
 * (qraf_hip_set_qgemm_tuning) selects the uniform grid.  Affects the
 * workspace queries too.  No counterpart in the reference (a performance
 * knob). */
int qraf_hip_set_qgemm_schedule(int32_t mode, int32_t min_blocks);
/* Wave-split form of the tile-major GEMM (each workgroup's 4 waves take its
 * quant blocks in turn and meet once in LDS at the end): mode 1 selects it
 * for every tiled batch over 16 rows, -1 never, 0 (the default) for batches
 * of 17-32 rows and of 33-64 rows below 16384 output rows, unless
 * qraf_hip_set_qgemm_tuning forces another form;
 * tiles_per_workgroup 2, 3 or 4 fixes its 16-row weight tiles per workgroup
 * (0: automatic).  Affects the workspace queries and the SwiGLU-epilogue
 * entry point too.  No counterpart in the reference (a performance knob). */
int qraf_hip_set_qgemm_kw(int32_t mode, int32_t tiles_per_workgroup);
/* Workspace (bytes) that lets qraf_hip_qgemm_dev split the in_dim range of an
 * out_dim x in_dim product at this batch across workgroups; 0 when it does
 * not split. */
uint64_t qraf_hip_qgemm_workspace_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim, int32_t batch);
/* dispatch_matvec_q (backend.cpp:131-199) for `batch` activation rows at
 * once on the matrix cores: y[m][i] = dot(row_i(w), x[m]) (+ add[m][i] when add
 * is not NULL; add may equal y), m < batch, i < out_dim.  w: Q8_0 (4-byte
 * aligned) or Q4_0 (2-byte aligned), block size 32, in_dim a multiple of 32;
 * x given as the hi/lo planes of qraf_hip_split_bf16_dev (16-byte aligned).
 * workspace (16-byte aligned, no initialisation needed) of at least
 * qraf_hip_qgemm_workspace_bytes enables the split-K path; NULL runs one
 * split.  The split-K sum is taken in a fixed order: results are
 * deterministic.  Calls that share a workspace must not overlap.
 * Error bound per output: sum_k |w_k| (2^-20 |x_k| + 2^-25)
 * + (in_dim+2) 2^-24 sum_k |w_k x_k|, for |x_k| < 2^24. */
int qraf_hip_qgemm_dev(const void* w, uint32_t dtype, uint32_t block_size, uint32_t out_dim, uint32_t in_dim,
                       const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, float* y, const float* add,
                       void* workspace, uint64_t workspace_bytes, void* stream);
/* Tile-major copy of a Q8_0/Q4_0 matrix (block size 32), the weight operand of
 * qraf_hip_qgemm_tiled_dev: for every 16-row tile and quant block, the 16
 * block scales then the 16 rows' 32 quants (rows past out_dim are zero), so a
 * wavefront's weight loads are contiguous.  The same bytes as the reference
 * layout (quantize.h:11-30), reordered; no counterpart in the reference. */
uint64_t qraf_hip_tiled_weight_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim);
int qraf_hip_repack_tiles_dev(const void* w, uint32_t dtype, uint32_t out_dim, uint32_t in_dim, void* dst,
                              void* stream);
/* qraf_hip_qgemm_dev on a tile-major weight copy (16-byte aligned), with its
 * own split-K workspace size (batches over 32 rows run a pipelined kernel
 * with 256-row weight tiles). */
uint64_t qraf_hip_qgemm_tiled_workspace_bytes(uint32_t dtype, uint32_t out_dim, uint32_t in_dim, int32_t batch);
int qraf_hip_qgemm_tiled_dev(const void* w_tiled, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                             const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, float* y, const float* add,
                             void* workspace, uint64_t workspace_bytes, void* stream);
/* Greedy LM head without logits: tokens[b] = Sampler::argmax
 * (sampler.cpp:25-35: the first of the largest values) of row b of
 * qraf_hip_qgemm_tiled_dev's product (out_dim = vocabulary rows), the product
 * never written.  Where the tiled plan for this shape is the pipelined kernel
 * it runs unsplit, each workgroup writing its best (value, index) per row to
 * keys (8-byte aligned, at least qraf_hip_qgemm_tiled_argmax_keys_bytes), and
 * a second launch reduces them: *fused = 1.  Otherwise nothing is launched
 * and *fused = 0 (the caller then takes the argmax of the written product).
 * A row holding NaN takes the largest of its numbers (the reference keeps a
 * NaN at position 0).  No counterpart in the reference (a fusion of the
 * logits projection and Sampler::argmax). */
uint64_t qraf_hip_qgemm_tiled_argmax_keys_bytes(uint32_t out_dim, int32_t batch);
int qraf_hip_qgemm_tiled_argmax_dev(const void* w_tiled, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                                    const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, void* keys,
                                    uint64_t keys_bytes, uint32_t* tokens, int32_t* fused, void* stream);

/* The SwiGLU front of mlp_forward (attention.cpp:172-178) fused into the
 * tile-major GEMM: w_tiled's rows interleave the gate and up projections (row
 * 2i = gate_i, row 2i+1 = up_i, out_dim = 2F, even); out_hi/out_lo [batch][F]
 * receive silu(gate) * up as the hi/lo planes the down projection's GEMM
 * reads (qraf_hip_split_bf16_dev form; they must not overlap x_hi/x_lo).
 * The pipelined kernel runs unsplit (128 weight rows x 64 batch rows per
 * workgroup), so no workspace is needed and the gate/up sums never leave the
 * registers; the sums are those of qraf_hip_qgemm_tiled_dev in the same form.
 * No counterpart in the reference (a fusion of two of its steps). */
int qraf_hip_qgemm_tiled_silu_dev(const void* w_tiled, uint32_t dtype, uint32_t out_dim, uint32_t in_dim,
                                  const uint16_t* x_hi, const uint16_t* x_lo, int32_t batch, uint16_t* out_hi,
                                  uint16_t* out_lo, void* stream);

/* ------------------------------------------------------------- engine */

/* The model hyper-parameters the reference reads from the QRAF config block
 * (loader.cpp:151-177, types.h:97-124).  num_kv_heads 0 means num_heads;
 * head_dim = hidden_size / num_heads (16, 32, 64 or 128). */
typedef struct qraf_model_config {
    uint32_t vocab_size, hidden_size, num_layers, num_heads, num_kv_heads, intermediate_size, max_seq_len;
    float rope_theta, rms_norm_eps;
} qraf_model_config;

/* Engine resources.  kv_dtype F32 (0, the reference's KVCache), F16, or I8
 * (QuantizedKVCache; head_dim 64/128, page_size % 4 == 0);
 * page_size tokens per KV page (0 -> 16, must divide 256); max_batch rows
 * per step (0 -> 1, at most 1024); num_pages KV pages per layer (0 -> enough
 * for max_batch sequences of min(max_seq_len, 8192) positions). */
typedef struct qraf_engine_options {
    uint32_t kv_dtype, page_size, max_batch, num_pages;
} qraf_engine_options;

typedef struct qraf_engine qraf_engine;

int qraf_engine_create(const qraf_model_config* config, const qraf_engine_options* options, qraf_engine** engine);
int qraf_engine_destroy(qraf_engine* engine);
/* Transformer::init weight binding (transformer.cpp:96-126, :310-400) for
 * one tensor, by the reference's names: model.embed_tokens.weight,
 * lm_head.weight (absent: tied to the embedding), model.norm.weight,
 * model.layers.<l>.{self_attn.{q,k,v,o}_proj.weight, self_attn.{q,k,v}_proj.bias,
 * mlp.{gate,up,down}_proj.weight, input_layernorm.weight,
 * post_attention_layernorm.weight}.  Shapes follow the reference's
 * [out, in] orientation; data is host memory, copied to HBM.  Quantized
 * tensors need block size 32; biases that are not F32 are ignored and the
 * four attention (three MLP) matrices of a layer must share one dtype, as in
 * the reference; other names are ignored. */
int qraf_engine_set_tensor(qraf_engine* engine, const char* name, uint32_t dtype, uint32_t block_size,
                           const uint32_t* shape, uint32_t ndim, const void* data, uint64_t bytes);
/* All weights synthetic, generated on the device: every tensor N(0, 0.02)
 * from qraf_hip_gen_weights_dev with stream = qraf_hip_name_hash(name),
 * norms 1, optional F32 q/k/v biases, lm_head unless tied. */
int qraf_engine_generate_weights(qraf_engine* engine, uint32_t weight_dtype, uint32_t embed_dtype,
                                 uint32_t head_dtype, int32_t tied, int32_t qkv_bias, uint64_t seed);
/* Checks that every tensor the forward pass reads is present. */
int qraf_engine_finalize(qraf_engine* engine);

/* Sampler on the device (src/sampling/sampler.cpp).  Parameters as in
 * SamplingConfig (include/sampling/sampler.h:10-17): temperature <= 0 is
 * greedy (Sampler::argmax, :25-35); otherwise p = logit / temperature, the
 * top_k largest (all when top_k <= 0 or >= vocab), softmax over them, the top_p nucleus when 0 < top_p < 1,
 * and the first candidate whose cumulative probability reaches the row's
 * uniform (Sampler::sample, :57-128).  repetition_penalty != 1 first applies
 * Sampler::apply_repetition_penalty (:37-49) in place to each row with that
 * row's recent tokens.  The uniform of a row is the draw the reference's
 * std::mt19937 would make (std::uniform_real_distribution<float>(0, 1)); the
 * host supplies it, so that the stream of draws follows the reference's. */
typedef struct qraf_sampling_params {
    float temperature;
    int32_t top_k;
    float top_p;
    float repetition_penalty;
} qraf_sampling_params;

/* Device pointers, stream-ordered: logits [rows][vocab] (penalised in
 * place), recent [rows][recent_stride] with recent_count [rows] valid
 * entries (may be NULL when repetition_penalty is 1), uniforms [rows] (may
 * be NULL when greedy), tokens [rows] out.  No device scope synchronisation.
 * Every top_k (<= 0 or >= vocab: the whole vocabulary).  Candidate lists of
 * at most 4096 tokens are sorted in on-chip memory; a whole-vocabulary row
 * is reproduced exactly from the tokens whose exp(p - max) terms are not
 * absorbed by the reference's sequential fp32 sums.  Larger candidate lists
 * (4096 < top_k < vocab, or more than 4096 unabsorbed tokens) are sorted in
 * sort storage of rows * vocab * 16 bytes that the library allocates on the
 * device's first such call (temperature > 0 and top_k outside 1..4096),
 * grows as needed and holds until the process ends; that first call must
 * not be made under stream capture (QRAF_HIP_ERR_STATE). */
int qraf_hip_sample_dev(float* logits, int32_t rows, int32_t vocab, const qraf_sampling_params* params,
                        const uint32_t* recent, const int32_t* recent_count, int32_t recent_stride,
                        const float* uniforms, uint32_t* tokens, void* stream);

/* QRAF file -> HBM.  The file layout of include/qraf/format.h:26-132 is
 * checked as validate_header (src/qraf/header.cpp:8-45) and get_string
 * (src/qraf/loader.cpp:273-277) do, and strings must end inside the string
 * table; a malformed file returns QRAF_HIP_ERR_FORMAT, an unreadable path
 * QRAF_HIP_ERR_INVALID.
 *
 * qraf_file_read_config: the model config stored in the file
 * (QrafModel::parse_config, loader.cpp:133-177), with ModelConfig's defaults
 * (include/core/types.h:97-124) for absent keys.  Host only: no GPU use.
 * num_tensors may be NULL.
 *
 * qraf_engine_create_from_file: QrafModel::load + Transformer::init
 * (loader.cpp:51-117, src/nn/transformer.cpp:310-439) in one call: maps the
 * file, creates an engine with the file's config and `options`, copies every
 * tensor from the mapping into HBM (qraf_engine_set_tensor) and finalizes.
 * Runs the LLaMA-family architectures (llama, qwen2, mistral, or none named);
 * others return QRAF_HIP_ERR_INVALID.  *engine is NULL on failure. */
int qraf_file_read_config(const char* path, qraf_model_config* config, uint32_t* num_tensors);
int qraf_engine_create_from_file(const char* path, const qraf_engine_options* options, qraf_engine** engine);

/* Sequences own KV pages; positions are added in order (pos <= length). */
int qraf_engine_seq_create(qraf_engine* engine, int32_t* seq_id);
int qraf_engine_seq_release(qraf_engine* engine, int32_t seq_id);
int qraf_engine_seq_length(qraf_engine* engine, int32_t seq_id, int32_t* length);
int qraf_engine_free_pages(qraf_engine* engine, int32_t* free_pages);

/* One batched decode step: row i feeds token tokens[i] at position
 * positions[i] of sequence seq_ids[i] (a sequence may own several rows, in
 * increasing position order: chunked prefill).  Rows with want_logits[i] != 0
 * (all rows when want_logits is NULL) get logits, written compactly in row
 * order to logits [k][vocab] and/or their argmax (Sampler::argmax,
 * sampler.cpp:25-35) to next_tokens [k]; either output may be NULL.
 * QRAF_HIP_ERR_NOMEM when the KV page pool cannot hold the new positions (no
 * state changes in that case).  The reference has no batched call: this is
 * Transformer::forward (transformer.cpp:573-639) for many sequences at once. */
int qraf_engine_step(qraf_engine* engine, int32_t n_rows, const int32_t* seq_ids, const uint32_t* tokens,
                     const int32_t* positions, const uint8_t* want_logits, float* logits, uint32_t* next_tokens);
/* Pipelined greedy steps.  qraf_engine_step_async validates and issues one
 * step as qraf_engine_step does (argmax of the rows that want logits; their
 * logits stay in HBM) and returns without waiting for it.  Row i feeds
 * tokens[i], or, where token_src != NULL and token_src[i] >= 0, the greedy
 * token of logit row token_src[i] of the step issued just before this one,
 * taken on the device: a decode row need not wait for its previous token to
 * reach the host, so the host builds step N+1 while step N runs.  At most two
 * steps are in flight (QRAF_HIP_ERR_STATE for a third);
 * qraf_engine_step_collect waits for the oldest and writes its greedy tokens
 * to next_tokens [k] (k = its rows that wanted logits, returned in *n_tokens;
 * either may be NULL).  qraf_engine_step and qraf_engine_forward return
 * QRAF_HIP_ERR_STATE while steps are in flight; qraf_engine_sample and
 * qraf_engine_read_logits wait for every issued step and read the latest's
 * logits.  No reference counterpart: InferenceEngine::generate_tokens
 * (inference.cpp:68-159) and the scheduler feed each sampled token back from
 * the host, one step at a time. */
int qraf_engine_step_async(qraf_engine* engine, int32_t n_rows, const int32_t* seq_ids, const uint32_t* tokens,
                           const int32_t* token_src, const int32_t* positions, const uint8_t* want_logits);
int qraf_engine_step_collect(qraf_engine* engine, uint32_t* next_tokens, int32_t* n_tokens);
/* Steps are captured once per shape (rows, logit rows, head, context bound
 * rounded up to a power of two, kernel tuning) into a HIP graph and replayed
 * (on = 1, the default); on = 0 launches every step's kernels eagerly.  No
 * reference counterpart: an execution detail of qraf_engine_step. */
int qraf_engine_set_graphs(qraf_engine* engine, int32_t on);
/* keep = 0: a step that wants only greedy tokens (qraf_engine_step with
 * logits NULL and next_tokens set, qraf_engine_step_async) writes no logits:
 * where its head runs as the pipelined tile-major GEMM (more than 64 logit
 * rows at the usual vocabulary sizes) Sampler::argmax (sampler.cpp:25-35) is
 * taken in that GEMM's epilogue (qraf_hip_qgemm_tiled_argmax_dev), the same
 * tokens without the [rows][vocab] write and re-read; qraf_engine_sample and
 * qraf_engine_read_logits return QRAF_HIP_ERR_STATE after such a step.
 * keep = 1 (the default): every step leaves its logits in HBM.  No reference
 * counterpart: the reference's forward always returns the logits. */
int qraf_engine_set_keep_logits(qraf_engine* engine, int32_t keep);
/* Sampling of the last step's logit rows where they lie in HBM (the rows
 * that step returned logits or argmax for, in order; row0 .. row0+rows-1 of
 * them): repetition penalty with each row's recent tokens (host arrays
 * [rows][recent_stride], recent_count [rows]; may be NULL when the penalty is
 * 1), then greedy or top-k/top-p sampling with the host uniforms [rows] (may
 * be NULL when greedy), as qraf_hip_sample_dev.  Only token ids and the
 * small host arrays cross PCIe. */
int qraf_engine_sample(qraf_engine* engine, int32_t row0, int32_t rows, const qraf_sampling_params* params,
                       const uint32_t* recent, const int32_t* recent_count, int32_t recent_stride,
                       const float* uniforms, uint32_t* tokens);
/* The last step's logit rows row0 .. row0+rows-1 (the rows it returned
 * logits or argmax for, in order) copied from HBM to out [rows][vocab]: a
 * step can keep its logits on the device and a caller read back only the
 * rows it inspects.  No reference counterpart (Transformer::forward returns
 * every logit by value, transformer.cpp:622-639). */
int qraf_engine_read_logits(qraf_engine* engine, int32_t row0, int32_t rows, float* out);
/* Host-side cost of qraf_engine_step / _step_async, accumulated since the last
 * reset: host_us = time from entry until every launch and copy of the step
 * was issued (validation, page bookkeeping, staging, graph launch), wait_us =
 * time blocked waiting for steps (qraf_engine_step's final synchronisation,
 * qraf_engine_step_collect).  No reference
 * counterpart (a measurement aid). */
typedef struct qraf_engine_stats {
    uint64_t steps, rows;
    double host_us, wait_us;
    /* steps launched eagerly, step graphs captured (each also launched),
     * step graph launches, and pad rows run (row padding, below) */
    uint64_t eager_steps, graph_captures, graph_launches, pad_rows;
} qraf_engine_stats;
int qraf_engine_get_stats(qraf_engine* engine, qraf_engine_stats* stats, int32_t reset);
/* Row padding of steps with step graphs on: a step of more than 8 rows runs
 * padded to a multiple of `rows` (at most max_batch), its logit rows too, so
 * that steps of nearby sizes replay one graph.  Pad rows use a scratch KV
 * page of their own and return nothing; results of real rows are the same
 * whatever the padding.  rows 1: off; default 16.  No reference counterpart
 * (a launch-cost measure). */
int qraf_engine_set_row_padding(qraf_engine* engine, int32_t rows);
/* Fusions that change how a step runs, not what it computes: bit 0
 * (default on) = one-row steps apply the QKV bias, RoPE and the K/V store
 * inside the QKV matvec (its one-shot form; f32 and fp16 pages) instead of a
 * separate launch (bit-identical either way); bit 1 (default on) = steps of
 * more than 256 rows run the gate/up GEMM unsplit with the SiLU-gate in its
 * epilogue (qraf_hip_qgemm_tiled_silu_dev) instead of split-K partials and
 * a separate SiLU/split launch (the same arithmetic summed in another order,
 * within the GEMM's error bound); bit 2 (default on) = steps of 2-8 rows
 * run each projection that qraf_hip_matvec_q_batch_dev covers with rows x
 * out_dim x in_dim at most 96 Mi (where it measured faster than the GEMM's
 * split, GEMM and reduction launches) on it, with the RMSNorm / SiLU-gate
 * formed in its staging; when the QKV and O projections qualify, the layer
 * runs projection by projection instead of as the split-K GEMM layer (fp32
 * products as at batch 1, summed in another order than the GEMM's).  No
 * reference counterpart (launch-count and traffic measures). */
int qraf_engine_set_fusion(qraf_engine* engine, int32_t flags);
/* Repetition penalty on the device for one sequence, set before its first
 * step (QRAF_HIP_ERR_STATE after): from then on every token the sequence is
 * fed (prompt rows, decode rows, tokens taken on the device from a previous
 * step's argmax) is counted on the device, and the greedy token of each of
 * its logit rows (next_tokens of qraf_engine_step, the tokens of
 * qraf_engine_step_async / _step_collect) is Sampler::argmax after
 * Sampler::apply_repetition_penalty (sampler.cpp:25-49) with the prompt and
 * every fed token as the recent list, as InferenceEngine::generate_tokens
 * builds it (inference.cpp:104-125): the same token as qraf_engine_sample with
 * that list, without the list crossing PCIe, so penalised greedy decoding
 * can run pipelined.  The logits the step leaves or returns stay
 * unpenalised.  penalty 1 turns it off.  At most 2 * max_batch penalised
 * sequences at a time (QRAF_HIP_ERR_NOMEM beyond); vocabularies that are a
 * multiple of 4 only (QRAF_HIP_ERR_INVALID otherwise).  The first call
 * allocates 2 * max_batch * vocab * 4 bytes of counts and drops the captured
 * step graphs.  No reference counterpart as an entry point. */
int qraf_engine_set_repetition_penalty(qraf_engine* engine, int32_t seq_id, float penalty);
/* Transformer::forward(token, pos) -> logits [vocab] (transformer.cpp:622-639)
 * on the engine's default sequence, and Transformer::reset() (:641-643). */
int qraf_engine_forward(qraf_engine* engine, uint32_t token, int32_t pos, float* logits);
int qraf_engine_reset(qraf_engine* engine);

#ifdef __cplusplus
}
#endif
#endif
