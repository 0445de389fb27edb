/*
 * fdattn.h -- C ABI of the MI355X (gfx950) split decode-attention library
 * (libfdattn.so).
 *
 * The library implements the three kernels of vllm_fastdecode's split
 * decode-attention path as hand-written HIP for CDNA4:
 *
 *   1. paged partial decode attention over a subset of a sequence's KV
 *      blocks, emitting (out, lse);
 *   2. the log-sum-exp merge of two partials (GPU tier + host tier);
 *   3. the reshape_and_cache slot-mapping write into a paged KV cache;
 *
 * plus the reference's host-core kernel itself (fd_host_decode_partial, x86
 * AVX-512/AVX2), so part of the host tier can be reduced by the host cores
 * while the GPU reads the rest.
 *
 * The same kernels serve both tiers of the reference's G+C block space: the
 * HBM tier (vLLM's [num_blocks, block_size, kv_heads, 2*head_size] cache) and
 * the host tier ([num_blocks, kv_heads, block_size, head_size] in pinned host
 * memory that the GPU reads and writes zero-copy). Layouts are described by
 * element strides, so one entry point covers both.
 *
 * Conventions shared by every entry point:
 *   - All buffers are caller-owned; nothing is allocated, and outputs are
 *     written in place (cpu_attn.cpp:452-489 and :491-517 contract).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and the call returns without synchronising (fd_host_decode_partial,
 *     which takes no stream, runs on the host and returns when done).
 *   - Arguments are validated on the host before any launch; an invalid call
 *     returns a non-zero status, writes nothing, and leaves a message for
 *     fd_last_error() (mirrors the TORCH_CHECKs of cpu_attn.cpp:433-477 and the
 *     "check every slot before any write" rule of cpu_attn.cpp:506-510).
 *   - Device pointers may point at HBM or at mapped pinned host memory
 *     (see fd_host_alloc / fd_host_device_pointer).
 *   - Strides are in elements, not bytes. The innermost (head_size)
 *     dimension must be contiguous and 16-byte aligned for the fast kernels,
 *     which take a block_size that is a multiple of 16 up to 1024, a
 *     head_size that is a multiple of 8 up to 256, fp16 / bf16 and
 *     num_heads / num_kv_heads up to 512; other shapes and layouts take a
 *     slower generic kernel.
 */
#ifndef FDATTN_H_
#define FDATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (the reference supports fp16, bf16 and fp32 KV:
 * cpu_attn.cpp:439-448). */
enum fd_dtype { FD_F16 = 0, FD_BF16 = 1, FD_F32 = 2 };

/* Status codes. */
enum fd_status {
  FD_OK = 0,
  FD_ERR_INVALID = 1,     /* bad shape, stride, dtype or pointer */
  FD_ERR_RANGE = 2,       /* slot or block id outside the cache */
  FD_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  FD_ERR_HIP = 4,         /* a HIP runtime call failed */
  FD_ERR_UNSUPPORTED = 5, /* valid but not implemented (e.g. head_size) */
  FD_ERR_RESOURCE = 6     /* the host ran out of memory or threads */
};

/* Message describing the last failed call on this host thread
 * (the reference reports errors as RuntimeError via TORCH_CHECK). */
const char* fd_last_error(void);

/* Library ABI version (bumped when a signature changes). */
int fd_abi_version(void);

/* ------------------------------------------------------------------------
 * Paged partial decode attention.
 *
 * Replaces both implementations of the partial in the reference:
 *   - the host-tier kernel decode_attn (fastdecode/csrc/cpu_attn.cpp:452-489,
 *     body :298-411), called at fastdecode/backend.py:350-351;
 *   - the GPU-tier FlashAttention paged decode
 *     (flash_attn_varlen_func with max_seqlen_q=1, return_softmax_lse=True,
 *     fastdecode/backend.py:305-316).
 *
 * For every sequence i < n and query head h < num_heads:
 *   out[i, h, :] = softmax(scale * q[i, h] . K_i^T) @ V_i
 *   lse[h, i]    = logsumexp(scale * q[i, h] . K_i^T)      (natural log)
 * over the lens[i] tokens held in blocks block_table[i, 0 .. ceil(lens[i] /
 * block_size)), in that order; only the last listed block may be partial and
 * no table entry past it is read. q head h attends kv head
 * h / (num_heads / num_kv_heads). A row with lens[i] <= 0 yields out = 0 and
 * lse = -inf (cpu_attn.cpp:324-331). Accumulation is fp32.
 *
 * q           [n, num_heads, head_size], dtype kv_dtype, strides
 *             (q_stride_seq, q_stride_head, 1)
 * k_cache,
 * v_cache     paged caches of kv_dtype; token t of block b, kv head g starts
 *             at b*kv_stride_block + g*kv_stride_head + t*kv_stride_token.
 *             Host tier [C, KVH, BS, D]: (KVH*BS*D, BS*D, D).
 *             vLLM HBM tier [B, BS, KVH, 2D] K/V halves: (BS*KVH*2D, 2D, KVH*2D).
 * num_blocks  blocks in the cache; a table entry outside [0, num_blocks) or
 *             lens[i] > bt_width*block_size is a device-side range error: the
 *             row's out and lse become NaN instead of reading out of bounds.
 * block_table int32 [n, >= bt_width], row stride bt_stride. The launch is
 *             planned for rows of up to bt_width blocks: a caller whose table
 *             is sized to the cache's capacity passes bt_width =
 *             ceil(longest row / block_size) (flash-attn's max_seqlen_k) with
 *             the full row stride, and pays nothing for the unused columns.
 * lens        int32 [n]
 * row_order   optional int32 [n] permutation of 0..n-1 (may be NULL): the order
 *             in which rows are scheduled. Results do not depend on it; passing
 *             rows longest-first shortens the launch's tail when lengths vary.
 *             No counterpart in the reference (its planner knows every length
 *             on the host, fastdecode/plan.py:103-199). Entries outside
 *             [0, n) are skipped.
 * out         [n, num_heads, head_size] of out_dtype (kv_dtype or FD_F32),
 *             strides (out_stride_seq, out_stride_head, 1)
 * lse         fp32, lse[h, i] at h*lse_stride_head + i
 * workspace   device scratch of >= fd_paged_decode_workspace_size(...) bytes
 *             (may be NULL when that size is 0). Launches on one stream may
 *             share it; launches that may overlap (other streams) need one
 *             each. Its contents need no clearing between calls.
 * ------------------------------------------------------------------------ */
int fd_paged_decode_partial(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const void* k_cache, const void* v_cache,
    int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks,
    const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens, const int32_t* row_order,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype,
    float* lse, int64_t lse_stride_head,
    void* workspace, size_t workspace_bytes,
    void* stream);

/* fd_paged_decode_partial for a caller that knows the rows' token total
 * (the sum of lens over the n rows; a serving step's scheduler has it on the
 * host). The launch plan otherwise sees only the table width; the total
 * gives the rows' mean fill of bt_width * block_size, which selects three
 * plans that cut rows into more tasks:
 *   - rows of uneven length (fill below 0.8) on the matrix-core kernel with
 *     16 heads per task, at up to 1.5 rows per CU: tasks that fill three
 *     workgroups per CU ("slot fill");
 *   - full rows (fill 0.8 or more) at 2.0-2.6 (sequence, kv head) rows per
 *     CU and D = 128: half-row tasks;
 *   - all but equal rows (fill 0.95 or more) at D = 64: quarter-row tasks at
 *     1.0-1.3 rows per CU and half rows at 2.0-2.6.
 * Results agree with fd_paged_decode_partial's within rounding: a different
 * task split sums the fp32 partials in a different order, so hinted and
 * unhinted calls are not bit-identical. total_tokens = 0: unknown (the same
 * plan as fd_paged_decode_partial); a wrong total costs time, never
 * correctness. No counterpart in the reference: its FlashAttention call
 * plans from max_seqlen_k alone (fastdecode/backend.py:306-314). */
int fd_paged_decode_partial_hint(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const void* k_cache, const void* v_cache,
    int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks,
    const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens, const int32_t* row_order,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype,
    float* lse, int64_t lse_stride_head,
    void* workspace, size_t workspace_bytes,
    void* stream, int64_t total_tokens);

/* Measurement helper: fd_paged_decode_partial (same arguments, same results)
 * that also records when each workgroup of the decode launch reaches a few
 * points, for launches that take the 16-bit VALU kernel (otherwise
 * FD_ERR_UNSUPPORTED, nothing launched). timeline: a device buffer of
 * timeline_workgroups * 8 uint64 (16-byte aligned, zeroed by the caller);
 * a launch of more workgroups is FD_ERR_INVALID. Words of workgroup w, at
 * timeline[8 w ...], in ticks of the GPU's 100 MHz real-time counter
 * (s_memrealtime): 0 task start, 1 wave 0's block ids in registers, 2-5 each
 * wave's end of its block loop, 6 the task's end (its result stored); word 7
 * packs the task's block count (bits 0-15), its working waves (16-23) and
 * its sequence (32-63). Workgroups with nothing to do leave their words
 * unwritten. No counterpart in the reference; it splits a launch's time into
 * start-up, streaming and drain. */
int fd_paged_decode_timeline(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const void* k_cache, const void* v_cache,
    int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks,
    const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens, const int32_t* row_order,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype,
    float* lse, int64_t lse_stride_head,
    void* workspace, size_t workspace_bytes,
    void* stream, uint64_t* timeline, int64_t timeline_workgroups);

/* Bytes of workspace fd_paged_decode_partial (and _hint, whatever its token
 * total) needs for these sizes (the block-range split partials), whatever
 * the kv dtype and wherever the cache lies: the largest need of the kernels
 * such a call may take (an fp32 cache streams twice the bytes per block and
 * may split rows sooner). No counterpart in the reference: its CPU kernel
 * keeps per-thread scratch in std::vector (cpu_attn.cpp:314-318). */
int fd_paged_decode_workspace_size(
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, int32_t bt_width, size_t* bytes);

/* Which kernel a decode launch of these sizes takes, and how it is cut into
 * tasks (the planner of fd_paged_decode_partial / fd_split_decode, on the
 * current device). No counterpart in the reference; for tests and for
 * integrators who want to know what runs.
 *   kv_dtype    FD_F16 / FD_BF16 / FD_F32
 *   aligned     1 if the launch meets the tiled kernels' alignment rules
 *               (16-byte aligned q, out and caches; strides multiples of 8
 *               elements), else 0 (the generic kernel)
 *   host_tier   1 if a tier lies in pinned host memory (16-bit launches then
 *               take the VALU kernel)
 *   total_tokens the rows' token total, as given to
 *               fd_paged_decode_partial_hint (0: unknown)
 * FD_DECODE_KERNEL and FD_SPLIT_BLOCKS are honoured as in a launch. */
#define FD_KERNEL_GENERIC 0 /* any layout, one wave per (sequence, head) */
#define FD_KERNEL_VALU 1    /* 16-bit KV, vector ALUs */
#define FD_KERNEL_MFMA 2    /* 16-bit KV, q.K on the matrix cores */
#define FD_KERNEL_MM 3      /* 16-bit KV, q.K and P.V on the matrix cores */
#define FD_KERNEL_F32 4     /* fp32 KV */

typedef struct {
  int32_t kernel;         /* FD_KERNEL_* */
  int32_t heads_per_task; /* query heads one task takes (its kernel's slots) */
  int32_t passes;         /* tasks per (sequence, kv head, block range) */
  int32_t split_blocks;   /* 16-token tiles per task */
  int32_t max_splits;     /* tasks per row at most (> 1: a combine pass) */
  int32_t wg_cap;         /* workgroups per compute unit the launch allows at most
                             (0: the kernel's own occupancy) */
  int32_t wave_blocks;    /* > 0: a task's four waves work only as far as its range
                             holds this many 16-token tiles each (a shorter range
                             works with fewer waves); 0: every wave works */
} FdDecodePlan;

int fd_decode_plan_info(int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                        int32_t block_size, int32_t bt_width, int32_t kv_dtype, int32_t aligned,
                        int32_t host_tier, int64_t total_tokens, FdDecodePlan* plan);

/* Size of the device scratch behind fd_paged_decode_partial_noalloc. */
#define FD_NOALLOC_SCRATCH_BYTES (32u << 20)

/* fd_paged_decode_partial without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc). No counterpart in the reference. Same arguments,
 * kernels and results as fd_paged_decode_partial; the split workspace is a
 * file-scope device array of FD_NOALLOC_SCRATCH_BYTES (32 MiB). Each GPU on
 * which the library's device code is loaded holds one such array until the
 * process ends, whether or not this entry point is ever called: every
 * process that runs the library's kernels on a GPU pays 32 MiB of its
 * memory for it. Sizes whose workspace
 * (fd_paged_decode_workspace_size) exceeds it are rejected with
 * FD_ERR_WORKSPACE before anything is written. The call allocates nothing.
 * Calls that may overlap on one GPU (other streams or threads) share the
 * array and race: serialise them, or use fd_paged_decode_partial with a
 * workspace each. The array needs no clearing between calls. */
int fd_paged_decode_partial_noalloc(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const void* k_cache, const void* v_cache,
    int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks,
    const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens, const int32_t* row_order,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype,
    float* lse, int64_t lse_stride_head,
    void* stream);

/* ------------------------------------------------------------------------
 * Fused split decode: both tiers of a row in one launch.
 *
 * Replaces the three calls of the reference's split-decode step
 * (fastdecode/backend.py:293-356): the GPU-tier FlashAttention partial
 * (:305-316), the host-tier decode_attn partial (:350-351) and
 * merge_attn_states (:354-355). For every sequence i and query head h the
 * result is attention over the union of the row's two block lists,
 *   out[i, h, :] = softmax(scale * q . [K_hbm ; K_host]^T) @ [V_hbm ; V_host]
 *   lse[h, i]    = logsumexp over both tiers (natural log),
 * which equals merge(partial_hbm, partial_host) of the separate calls. The
 * kernel walks each row's HBM-tier blocks, then its host-tier blocks, as one
 * list and merges in-kernel: no partial round trip and no merge launch.
 *
 * Each tier is described by an fd_kv_tier: the same cache/stride/table/length
 * conventions as fd_paged_decode_partial, per tier (tier-relative block ids,
 * as the reference's planner produces them: s_gpu_bt / s_gpu_lens and
 * s_cpu_bt / s_cpu_lens, fastdecode/plan.py:160-172). A row with no tokens in
 * either tier yields out = 0, lse = -inf; a range error in either tier makes
 * the row NaN. The host tier's caches may be mapped pinned host memory.
 * workspace: >= fd_paged_decode_workspace_size(n, ..., hbm->bt_width +
 * host->bt_width) bytes. No counterpart as a single call in the reference.
 * ------------------------------------------------------------------------ */
typedef struct fd_kv_tier {
  const void* k_cache;
  const void* v_cache;
  int64_t stride_block, stride_head, stride_token; /* elements */
  int64_t num_blocks;
  const int32_t* block_table; /* int32 [n, >= bt_width], row stride bt_stride */
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* lens; /* int32 [n]: tokens of each row held in this tier */
} fd_kv_tier;

int fd_split_decode(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const fd_kv_tier* hbm, const fd_kv_tier* host,
    const int32_t* row_order,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype,
    float* lse, int64_t lse_stride_head,
    void* workspace, size_t workspace_bytes,
    void* stream);

/* ------------------------------------------------------------------------
 * Device-side tier split of a decode step.
 *
 * The part of the reference's per-step planner build_host_plan
 * (fastdecode/plan.py:103-199, run on the host after a device-to-host copy of
 * the block table, fastdecode/backend.py:140-178) that a decode step needs,
 * computed on the GPU so the step needs no device-to-host copy. For every row
 * r < n_rows with seq_lens[r] tokens in blocks block_table[r, 0 .. nb):
 *   gpu_block_table[r, :] = its ids < num_gpu_blocks, in order, then zeros;
 *   cpu_block_table[r, :] = its ids >= num_gpu_blocks minus num_gpu_blocks,
 *                           in order, then zeros  (plan.py:82-100);
 *   gpu_lens[r], cpu_lens[r] = tokens held by each tier's blocks, the row's
 *                           last block holding L - (nb-1)*block_size
 *                           (plan.py:165-170).
 * For every token t < n_tokens (plan.py:150-152):
 *   gpu_slot_mapping[t]  = -1 for a host slot (>= num_gpu_blocks*block_size),
 *                          else slot_mapping[t];
 *   host_slot_mapping[t] = slot - num_gpu_blocks*block_size for a host slot,
 *                          else -1.
 * A host id past num_gpu_blocks + num_cpu_blocks, a host slot past
 * (num_gpu_blocks + num_cpu_blocks) * block_size, or a length needing more
 * than bt_width blocks, adds to *error_count (may be NULL) -- the planner's
 * RuntimeError and store_kv's range check, reported asynchronously; such a
 * row's lengths or ids make the decode kernels write NaN for it, and passing
 * error_count as fd_reshape_and_cache's write_gate keeps the step's KV
 * writes out of both tiers. The outputs have width
 * out_width >= bt_width and row stride out_stride. Feeding both tables to
 * fd_split_decode (HBM tier, host tier) decodes every row, P and S alike.
 * ------------------------------------------------------------------------ */
int fd_plan_tiers(
    const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* seq_lens, int32_t n_rows,
    int32_t num_gpu_blocks, int64_t num_cpu_blocks, int32_t block_size,
    int32_t* gpu_block_table, int32_t* cpu_block_table,
    int64_t out_stride, int32_t out_width,
    int32_t* gpu_lens, int32_t* cpu_lens,
    const int64_t* slot_mapping, int32_t n_tokens,
    int64_t* gpu_slot_mapping, int64_t* host_slot_mapping,
    int32_t* error_count, void* stream);

/* ------------------------------------------------------------------------
 * Log-sum-exp merge of two partials.
 *
 * Replaces vLLM's merge_attn_states(out, o_a, lse_a, o_b, lse_b) called at
 * fastdecode/backend.py:53-55,354-355, with the rule of the reference's torch
 * restatement merge_partials_torch (fastdecode/cpu_ops.py:93-113):
 *   lse := -inf where lse == +inf (FlashAttention's "empty");
 *   m = max(lse_a, lse_b); both empty => m = 0 and the weights' sum is 1,
 *   giving out = 0;
 *   w_x = exp(lse_x - m) / (exp(lse_a - m) + exp(lse_b - m));
 *   out = o_a * w_a + o_b * w_b   (fp32), converted to out_dtype.
 * out_lse (optional, may be NULL) receives m + log(sum of weights), i.e. the
 * lse of the merged partial (-inf when both are empty).
 * o_a, o_b and out are [n, num_heads, head_size] with strides
 * (stride_seq, stride_head, 1); lse_a, lse_b and out_lse are fp32 indexed
 * [h * lse_stride_head + i].
 * ------------------------------------------------------------------------ */
int fd_merge_attn_states(
    void* out, int64_t out_stride_seq, int64_t out_stride_head, int32_t out_dtype,
    const void* o_a, int64_t a_stride_seq, int64_t a_stride_head, int32_t a_dtype,
    const float* lse_a, int64_t lse_a_stride_head,
    const void* o_b, int64_t b_stride_seq, int64_t b_stride_head, int32_t b_dtype,
    const float* lse_b, int64_t lse_b_stride_head,
    float* out_lse, int64_t out_lse_stride_head,
    int32_t n, int32_t num_heads, int32_t head_size,
    void* stream);

/* ------------------------------------------------------------------------
 * reshape_and_cache: slot-mapping write of this step's K/V rows.
 *
 * Replaces vLLM's reshape_and_cache_flash (fastdecode/backend.py:49-51,
 * 270-273) for the HBM tier and the host-tier store_kv
 * (fastdecode/csrc/cpu_attn.cpp:491-517, body :413-431) for the pinned host
 * tier. For every token j < num_tokens with s = slot_mapping[j]:
 *   s < 0                 skipped (padding / other tier, plan.py:152);
 *   0 <= s < num_blocks*block_size
 *                         k_cache[s / block_size, token s % block_size, g, :]
 *                           = key[j, g, :]   for every kv head g (same for V);
 *   s >= num_blocks*block_size
 *                         not written; counted into *error_count when
 *                         error_count != NULL (a device int32).
 * write_gate (may be NULL): a device int32 written by earlier work on
 * `stream`, e.g. the error_count of fd_plan_tiers; when it is non-zero the
 * launch writes nothing, so a step whose slots the planner found past the
 * cache writes no KV at all (every slot checked before any write,
 * cpu_attn.cpp:506-510). It must not be the same counter as error_count.
 * The copy is bit-exact. key/value strides are per token and per head
 * (the rows may be strided views of a fused qkv tensor).
 * cache strides: element offset of (block b, token t, head g) is
 *   b*cache_stride_block + t*cache_stride_token + g*cache_stride_head.
 * slot_mapping is int64 and must be device-readable.
 * ------------------------------------------------------------------------ */
int fd_reshape_and_cache(
    const void* key, int64_t key_stride_tok, int64_t key_stride_head,
    const void* value, int64_t value_stride_tok, int64_t value_stride_head,
    void* k_cache, void* v_cache,
    int64_t cache_stride_block, int64_t cache_stride_token,
    int64_t cache_stride_head, int64_t num_blocks,
    const int64_t* slot_mapping, int32_t num_tokens,
    int32_t num_kv_heads, int32_t head_size, int32_t block_size,
    int32_t dtype, int32_t* error_count, const int32_t* write_gate,
    void* stream);

/* Host-side range check of host-resident slots before a write, the rule of
 * cpu_attn.cpp:506-510: every slot must lie in [0, capacity). Returns FD_OK,
 * or FD_ERR_RANGE with *first_bad (if not NULL) set to the first offending
 * index. Pure host code; never touches the GPU. */
int fd_check_slots(const int64_t* slots, int64_t m, int64_t capacity,
                   int64_t* first_bad);

/* ------------------------------------------------------------------------
 * Pinned host memory for the host tier.
 *
 * The reference keeps the host tier in pageable torch.zeros tensors and
 * stages every per-layer transfer through pinned buffers
 * (fastdecode/state.py:66-71, :93-124). Here the tier itself is allocated
 * pinned and mapped (hipHostMalloc), so the kernels above read and write it
 * directly over the link with no staging copy.
 * ------------------------------------------------------------------------ */
int fd_host_alloc(size_t bytes, void** host_ptr);
/* Frees a block made by fd_host_alloc (NULL: no-op; any other pointer is
 * FD_ERR_INVALID). It first waits for the work enqueued on the device that
 * was current at fd_host_alloc (hipDeviceSynchronize on that device only;
 * no other device is touched), so kernels still reading or writing the
 * block over the link finish before it goes; a caller that also uses the
 * block from other devices synchronises those first. Not to be called
 * during a stream capture: the wait then fails, the block is kept and the
 * call returns FD_ERR_HIP with "block kept" in fd_last_error(). */
int fd_host_free(void* host_ptr);
/* Device address of a pinned allocation made by fd_host_alloc. */
int fd_host_device_pointer(void* host_ptr, void** device_ptr);

/* ------------------------------------------------------------------------
 * Host-core partial decode attention (the co-processing leg of the split step).
 *
 * Replaces the reference's host-tier kernel decode_attn
 * (fastdecode/csrc/cpu_attn.cpp:452-489, body :298-411), called at
 * fastdecode/backend.py:350-351, with the same arguments and results as
 * fd_paged_decode_partial -- except that every pointer is a HOST address
 * (q, caches, table, lengths, out, lse) and the call runs synchronously on
 * the calling thread plus a persistent pool of num_threads - 1 workers
 * (0: one per CPU of the process's affinity mask, or FASTDECODE_CPU_THREADS;
 * at most FD_HOST_MAX_THREADS, larger counts are FD_ERR_INVALID).
 * Rows with lens <= 0 give out = 0, lse = -inf; a range error makes the row
 * NaN. Used to give part of each row's host-tier blocks to the host cores
 * while the GPU reads the rest over the link; the two partials are then
 * merged with fd_merge_attn_states. Needs AVX2, FMA and F16C
 * (FD_ERR_UNSUPPORTED otherwise). Calls are serialised per process.
 * ------------------------------------------------------------------------ */
int fd_host_decode_partial(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const void* k_cache, const void* v_cache,
    int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks,
    const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype,
    float* lse, int64_t lse_stride_head,
    int32_t num_threads);

/* fd_host_decode_partial in the background: checks the arguments as
 * fd_host_decode_partial does (an invalid call returns its error here and
 * queues nothing), queues the call for a runner thread of the library and
 * returns at once with *call, an id for fd_host_decode_wait. The runner first
 * waits for ready_event (a hipEvent_t; NULL: none), e.g. one recorded behind
 * the copy of q to the host, then makes the call; queued calls run one at a
 * time in queue order. Every buffer must stay valid, and out / lse unread,
 * until fd_host_decode_wait(*call) has returned; every started call must be
 * waited for once. No counterpart in the reference, whose host-tier kernel
 * runs synchronously inside the forward (fastdecode/backend.py:343-351); for
 * callers that overlap the host cores' share with the GPU's work (the hybrid
 * split) without a thread of their own. */
int fd_host_decode_partial_start(
    void* ready_event,
    const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const void* k_cache, const void* v_cache,
    int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks,
    const int32_t* block_table, int64_t bt_stride, int32_t bt_width,
    const int32_t* lens,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    void* out, int64_t out_stride_seq, int64_t out_stride_head,
    int32_t out_dtype,
    float* lse, int64_t lse_stride_head,
    int32_t num_threads, int64_t* call);

/* Blocks until the call queued as `call` has run and returns its status (the
 * message of a failure for fd_last_error() on this thread). *seconds (may be
 * NULL) = the time the call itself took, from the end of the wait for its
 * event. An id that is not pending (never started, or already waited for)
 * is FD_ERR_INVALID. */
int fd_host_decode_wait(int64_t call, double* seconds);

/* Worker count fd_host_decode_partial uses when num_threads is 0: the count
 * set by fd_host_set_threads, else FASTDECODE_CPU_THREADS, else one per CPU
 * of the process's affinity mask. Replaces the extension's get_num_threads
 * (cpu_attn.cpp:36-40,523). */
int fd_host_decode_threads(void);

/* Sets that count for the process (n <= 0 restores the default; n above
 * FD_HOST_MAX_THREADS is FD_ERR_INVALID). Replaces the extension's
 * set_num_threads (cpu_attn.cpp:521). */
int fd_host_set_threads(int32_t n);

/* Upper bound on the host-core worker count (a FASTDECODE_CPU_THREADS above
 * it is clamped). */
#define FD_HOST_MAX_THREADS 1024

/* Division of each row's host-tier blocks between the GPU and the host cores
 * for the hybrid split (host code; no counterpart in the reference, whose
 * host cores take every host block, i.e. cpu_fraction = 1). For row r with
 * nb = ceil(host_lens[r] / block_size) blocks, the host cores get its last
 * k = min(floor(nb * cpu_fraction + 1/2), nb) blocks and the GPU the rest:
 *   gpu_lens[r] = k ? (nb - k) * block_size : host_lens[r]  (whole blocks),
 *   cpu_lens[r] = host_lens[r] - gpu_lens[r],
 *   cpu_bt[r, 0 .. k) = host_bt[r, nb - k .. nb), then zeros up to bt_width.
 * The GPU keeps host_bt itself. *cpu_width (may be NULL) = the largest k.
 * A row needing more than bt_width blocks is FD_ERR_INVALID. */
int fd_share_host_blocks(const int32_t* host_bt, int64_t bt_stride, int32_t bt_width,
                         const int32_t* host_lens, int32_t n, int32_t block_size,
                         double cpu_fraction, int32_t* gpu_lens, int32_t* cpu_bt,
                         int64_t cpu_bt_stride, int32_t* cpu_lens, int32_t* cpu_width);

/* The host cores' share of a hybrid split step, started in one call (no
 * counterpart in the reference, whose host cores take the whole host tier
 * synchronously after staging q, fastdecode/backend.py:343-351). In order:
 *   1. enqueues on `stream` the copy of q (the GPU's [n, H, D], contiguous,
 *      kv_dtype) to q_host (pinned host memory of the same layout) and
 *      records ready_event (a hipEvent_t) behind it;
 *   2. divides each row's host-tier blocks as fd_share_host_blocks does
 *      (writes gpu_lens, cpu_bt, cpu_lens; cpu_bt's rows hold
 *      max(bt_width, 1) ids, cpu_bt_stride apart);
 *   3. queues, as fd_host_decode_partial_start does, fd_host_decode_partial
 *      over the host cores' blocks (q_host, cpu_bt, cpu_lens) into out (fp32
 *      [n, H, D], contiguous) and lse (fp32 [H, n], contiguous) behind
 *      ready_event, and returns at once with *call for fd_host_decode_wait.
 * The arguments are checked first (an invalid call enqueues and queues
 * nothing; host_bt may be NULL when bt_width is 0); a table row needing
 * more than bt_width blocks fails in step 2, after the copy was enqueued,
 * and queues no call. n = 0: nothing is done
 * and *call = 0 (nothing to wait for). Replaces the copy, the share and the
 * start that a caller would otherwise make one by one, which cost the step
 * ~0.1 ms of host time between the host cores' shares. */
int fd_hybrid_share_start(
    void* stream, void* ready_event, const void* q, void* q_host,
    const int32_t* host_bt, int64_t bt_stride, int32_t bt_width,
    const int32_t* host_lens, double cpu_fraction,
    int32_t* gpu_lens, int32_t* cpu_bt, int64_t cpu_bt_stride, int32_t* cpu_lens,
    const void* k_cache, const void* v_cache,
    int64_t kv_stride_block, int64_t kv_stride_head, int64_t kv_stride_token,
    int64_t num_blocks,
    int32_t n, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
    int32_t block_size, float scale, int32_t kv_dtype,
    float* out, float* lse, int32_t num_threads, int64_t* call);

/* Host-tier slot write on the host cores: the reference's store_kv
 * (cpu_attn.cpp:491-517, body :413-431) with host pointers.
 *   cache[slot / BS][kv head][slot % BS][:] = k[j][kv head][:]  (and V)
 * for j < m. k, v [m, KVH, D] with strides (k_stride_tok, k_stride_head, 1);
 * caches [num_blocks, KVH, BS, D] of dtype with strides (block, head, token).
 * Every slot is checked against [0, num_blocks * block_size) before any
 * write: FD_ERR_RANGE ("CPU slot out of range") and nothing written
 * otherwise. Synchronous; bit-exact copies. */
int fd_host_store_kv(const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                     const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                     void* k_cache, void* v_cache, int64_t cache_stride_block,
                     int64_t cache_stride_head, int64_t cache_stride_token,
                     int64_t num_blocks, const int64_t* slots, int64_t m,
                     int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                     int32_t dtype);

/* Vector width in bits fd_host_decode_partial uses on this CPU: 512
 * (AVX-512F; bf16 KV scores by vdpbf16ps where AVX512_BF16 is present,
 * unless FASTDECODE_CPU_ISA=avx512), 256 (AVX2; also when
 * FASTDECODE_CPU_ISA=avx2), 0 (neither: the call fails with
 * FD_ERR_UNSUPPORTED). No counterpart in the reference (its kernel is
 * compiled for one ISA, cpu_attn.cpp:1-40). */
int fd_host_decode_isa(void);

/* Measurement helper: reads `bytes` (a multiple of 64) of host memory at src
 * (64-byte aligned) on num_threads host cores (0: as fd_host_decode_partial
 * picks them), in 1 MiB pieces, each read as four interleaved streams of
 * prefetched 32-byte loads (one stream per core reads DRAM at about half
 * its rate on some hosts), with no work per byte beyond
 * an XOR into *checksum (the XOR of all 64-bit words). Its rate is what the
 * host cores can stream from DRAM: the bound of the host-core leg of the
 * split step. No counterpart in
 * the reference, whose README bounds the CPU side by the host's memory
 * bandwidth (README.md:86-87). */
int fd_host_stream_read(const void* src, size_t bytes, int32_t num_threads, uint64_t* checksum);

/* ------------------------------------------------------------------------
 * Measurement helper: streams `bytes` (a multiple of 16) from src to dst with
 * the same 16-byte vector loads the attention kernel uses. Used to calibrate
 * the HBM-traffic counters and the achievable copy bandwidth. No counterpart
 * in the reference.
 * ------------------------------------------------------------------------ */
int fd_stream_copy(void* dst, const void* src, size_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FDATTN_H_ */
