/* C ABI of the MI355X fused whole-model decode step (libmsdecode.so, gfx950).
 *
 * Every entry point takes plain device pointers and sizes, runs on the caller's
 * HIP stream and returns 0 on success or a negative MSD_E* code.  Apart from
 * msd_workspace_acquire, nothing here allocates device memory: buffers are sized
 * with the msd_*_bytes/elems queries and owned by the caller.
 *
 * Reference interfaces replaced (zahlmann/transformer):
 *   msd_decode_step       <- kernels/multi_sm_decode.py:369-432
 *                            multi_sm_decode_nlayer(w, config, token_id, pos, kv_packed)
 *                            and its launch jt.triton_call(_multi_sm_decode, ...) at :402-430
 *   msd_packed_weight_elems, msd_workspace_bytes
 *                         <- the packed_w size implied by kernels/fused_decode_nlayer.py:250-270
 *                            and the workspace layout of kernels/multi_sm_decode.py:390-400
 *   msd_sample_token      <- generate.py:28-65 sample_token(logits, temperature, top_p,
 *                            rep_penalty, generated_ids), with the np.random.choice draw
 *                            (generate.py:63,65) taken from a supplied uniform
 *   msd_sample_workspace_bytes
 *                         <- the host numpy temporaries of generate.py:28-65
 *   msd_prefill           <- model.py:194-231 prefill_with_kv(params, config, x) as used by
 *                            generate.py:70-90 (_prefill)
 *   msd_prefill_workspace_bytes
 *                         <- the activations XLA allocates for prefill_with_kv
 *   msd_tiles_bytes, msd_pack_tiles
 *                         <- no counterpart in the reference (its XLA prefill reads the f32
 *                            parameter arrays of model.py:194-231 as they are): a second copy
 *                            of the projection weights in matrix-core operand order
 *   msd_prefill_paged, msd_batch_decode_step, msd_batch_workspace_bytes
 *                         <- the batched decode over a paged KV cache that the reference
 *                            describes (PagePool with in-kernel page tables, batched decode
 *                            kernels: knowledge/program.md:214-216, 245-250); no code of it is
 *                            in the reference snapshot, so the interface is this library's own
 */
#ifndef MSDECODE_H
#define MSDECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model shape; same keys as the reference config dict (model.py:37-47). */
typedef struct msd_config {
  int32_t vocab_size;
  int32_t d_model;
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t n_layers;
  int32_t d_head;
  int32_t d_ff;
  int32_t context_len;
} msd_config;

enum {
  MSD_OK = 0,
  MSD_E_CONFIG = -1,      /* unsupported or inconsistent shape */
  MSD_E_ARG = -2,         /* null pointer, misaligned buffer, token/pos out of range */
  MSD_E_HIP = -3,         /* a HIP runtime call failed */
  MSD_E_TIMEOUT = -4,     /* a cross-workgroup wait exceeded its spin bound (reported by msd_check_status) */
};

/* Paths of the library (bits of msd_config_support). */
enum {
  MSD_PATH_DECODE = 1,    /* msd_decode_step / msd_decode_steps (the fused step) */
  MSD_PATH_PREFILL = 2,   /* msd_prefill, msd_prefill_paged, msd_pack_tiles */
  MSD_PATH_VERIFY = 4,    /* msd_verify */
  MSD_PATH_BATCHED = 8,   /* msd_batch_decode_step (any batch; a persistent launch where it fits) */
  MSD_PATH_SAMPLE = 16,   /* msd_sample_token (the vocabulary size) */
  MSD_PATH_BATCHED_STEP = 32,   /* msd_batch_decode_step runs up to 8 sequences as one persistent
                                   launch (on a device that holds its grid resident) */
};

/* The paths that accept cfg, as MSD_PATH_* bits (0 = none), or MSD_E_ARG for a null cfg.
 * n_workgroups is the decode grid the fused step would run on (msd_default_workgroups of the
 * device; 0 or less: 256, one per compute unit of an MI355X).  Makes no HIP call, so a host
 * can check a checkpoint's shape before touching the device.  Limits: d_head 64, n_heads a
 * multiple of n_kv_heads; the fused step needs one of the instantiated (d_model, d_ff) pairs
 * (see msd_decode_step) and context_len <= 2048; prefill d_model <= 1024 with d_model and
 * vocab_size multiples of 64 and d_ff of 32; verification and batched decode also
 * context_len <= 2048; the
 * sampler vocab_size <= 32768.  No counterpart in the reference (its Triton kernel takes any
 * shape through constexprs, kernels/multi_sm_decode.py:371-388): this library's shape query. */
int32_t msd_config_support(const msd_config* cfg, int32_t n_workgroups);

/* Kernel row layout: every row of K bf16 inputs is cut into blocks of 512 (the last block
 * holds the remaining S = 8*m values); within block b the value stored at offset
 * 512*b + 8*l + k (l < m, k < 8) is input element 512*b + k*m + l of the row.
 *
 * Number of bf16 elements of the packed per-layer weight buffer (kernel layout). */
int64_t msd_packed_weight_elems(const msd_config* cfg);

/* Bytes of device workspace a decode step needs for n_workgroups workgroups.
 * The workspace must be zero-filled once before first use; it is reused across steps. */
int64_t msd_workspace_bytes(const msd_config* cfg, int32_t n_workgroups);

/* Workgroups a step launches on device `device` (one per compute unit). */
int32_t msd_default_workgroups(int32_t device);

/* One fused decode step: embedding of the token, all layers (RMSNorm, QKV, RoPE, KV write
 * at `pos`, GQA attention over rows 0..pos, O projection, SwiGLU FFN, residuals), final
 * RMSNorm, tied logits over the vocabulary and argmax.
 *
 *   token_emb   bf16 (vocab_size, d_model), natural layout (embedding gather)
 *   output_proj bf16 (vocab_size, d_model): token_emb with every row in the kernel row layout
 *               (tied output projection; replaces the reference's output_proj_padded)
 *   packed_w    bf16, msd_packed_weight_elems(cfg) elements (kernel layout)
 *   lnf_s       bf16 (d_model) final RMSNorm scale
 *   rope        f32 (context_len, d_head): [cos(0..d_head/2) | sin(0..d_head/2)] per position
 *   token_id    input token, used when token_dev is NULL
 *   token_dev   optional device int32 holding the input token (e.g. the previous step's
 *               next_token), read by the kernel instead of token_id
 *   pos         position of the input token, 0 <= pos < context_len
 *   kv          bf16 KV cache [layer][K,V][kv_head][context_len][d_head], updated in place at pos
 *   workspace   msd_workspace_bytes(cfg, n_workgroups) bytes
 *   epoch       strictly increasing per call on one workspace (starts at 1)
 *   logits      f32 (vocab_size) output
 *   next_token  device int32[2] output: [0] argmax of logits (lowest index on ties),
 *               [1] the workspace status word at the end of the step (0 = ok; bit 0 = a
 *               cross-workgroup wait ran out, bit 1 = token_dev held an out-of-range id)
 *
 * Supported shapes: d_head 64 and (d_model, d_ff) one of (256, 704), (256, 768), (512, 1408),
 * (768, 2048), (1024, 2816) -- the reference's d_ff = 8 d / 3 rounded up to 128 (model.py:13-20)
 * for d_model 256..1024, and the tiny benchmark shape -- with any n_heads = d_model / 64,
 * n_kv_heads dividing n_heads, context_len up to 2048 (above 512 the attention of each head is
 * split over ceil(context_len / 512) workgroups) and n_workgroups no more than the device
 * holds at once (every workgroup waits on others; msd_default_workgroups is one per compute
 * unit).  Returns MSD_E_CONFIG otherwise.  Calls that share a workspace must be ordered on one
 * stream, and only one step may run on a device at a time (a concurrent kernel could keep some
 * of its workgroups from starting).
 */
int32_t msd_decode_step(const msd_config* cfg, const void* token_emb, const void* output_proj,
                        const void* packed_w,
                        const void* lnf_s, const float* rope, int32_t token_id,
                        const int32_t* token_dev, int32_t pos, void* kv, void* workspace,
                        uint32_t epoch, float* logits, int32_t* next_token,
                        int32_t n_workgroups, void* stream);

/* n_steps greedy decode steps in one launch: step s runs at position pos + s on the argmax of
 * step s - 1 (step 0 on token_id / token_dev), fed back on the device without leaving the
 * kernel.  Tags epoch .. epoch + n_steps - 1 (the next call on this workspace starts above
 * them).  tokens_out: device int32[2 * n_steps], (argmax, status) per step; logits:
 * n_steps x vocab_size f32 when all_logits != 0, else vocab_size (the last step's).  Other
 * arguments and requirements as msd_decode_step, with pos + n_steps <= context_len.
 * Replaces the persistent decode the reference describes (one launch for N steps with the
 * next token written in-kernel: knowledge/program.md:246-249, 441-444); no code of it is in
 * the reference snapshot. */
int32_t msd_decode_steps(const msd_config* cfg, const void* token_emb, const void* output_proj,
                         const void* packed_w, const void* lnf_s, const float* rope, int32_t token_id,
                         const int32_t* token_dev, int32_t pos, int32_t n_steps, void* kv,
                         void* workspace, uint32_t epoch, float* logits, int32_t all_logits,
                         int32_t* tokens_out, int32_t n_workgroups, void* stream);

/* Reads and clears the device status word of a workspace (synchronous on `stream`).
 * Returns MSD_OK, MSD_E_TIMEOUT when a wait of an earlier step ran out, or MSD_E_HIP. */
int32_t msd_check_status(void* workspace, void* stream);

/* A zero-filled decode workspace of `bytes` bytes on device `device`, in uncached device
 * memory: the exchange words the workgroups poll then bypass the L2 caches, which shortens
 * every cross-workgroup hop (any zero-filled device memory works; this is the fast kind).
 * Blocks come from a process-wide pool and are never freed (uncached memory must outlive
 * every kernel that read it): msd_workspace_release returns one to the pool, and a later
 * acquire of the same size on the same device re-zeroes and reuses it (after a device
 * synchronisation).  No counterpart in the reference (its exchange buffers are jax arrays,
 * kernels/multi_sm_decode.py:390-400).  Thread-safe.  MSD_E_ARG for bytes <= 0 or a NULL
 * `out`, MSD_E_HIP when the allocation fails. */
int32_t msd_workspace_acquire(int32_t device, int64_t bytes, void** out);
/* Returns a block from msd_workspace_acquire to the pool (MSD_E_ARG for an unknown pointer).
 * The caller must not use it afterwards; work still queued on it is waited for before reuse. */
int32_t msd_workspace_release(void* workspace);

/* Bytes of device workspace msd_sample_token needs for a vocabulary of `vocab` ids
 * (vocab <= 32768; MSD_E_CONFIG otherwise).  No initialisation is needed. */
int64_t msd_sample_workspace_bytes(int32_t vocab);

/* Draws the next token from f32 logits on the device, with numpy's arithmetic of the host
 * sampler reproduced (float32 penalty/temperature/softmax, numpy's pairwise sums, the
 * sequential float32 cumsum of the descending probabilities, a float64 inverse CDF):
 *
 *   temperature == 0      argmax of the penalised logits (lowest id on ties); no draw
 *   top_p >= 1            inverse CDF of the full softmax in id order
 *   top_p < 1             nucleus: ids sorted by descending probability (equal values in
 *                         ascending id order), kept up to and including the first whose
 *                         running float32 sum reaches top_p, renormalised, inverse CDF
 *
 *   seen         device uint8 (vocab): 1 for ids generated earlier in this sequence; the
 *                penalty (l / rep_penalty if l > 0 else l * rep_penalty) applies to them when
 *                rep_penalty != 1.  The drawn id is set to 1 on return.
 *   uniform      device float64: the draw u in [0, 1) (RandomState.random_sample()); may be
 *                NULL when temperature == 0
 *   token_out    device int32 output (can be the token input of the next msd_decode_step)
 *   probs_out    optional device f32 (vocab): the normalised probabilities in id order
 *                (temperature > 0)
 *   kept_out     optional device int32: number of ids the nucleus kept (top_p < 1)
 *   workspace    msd_sample_workspace_bytes(vocab) bytes, 256-byte aligned
 *
 * The exponential is the correctly rounded float32 value (numpy's float32 exp differs by up to
 * 2 ulp).  Calls sharing a workspace or `seen` must be ordered on one stream. */
int32_t msd_sample_token(const float* logits, int32_t vocab, double temperature, double top_p,
                         double rep_penalty, uint8_t* seen, const double* uniform,
                         int32_t* token_out, float* probs_out, int32_t* kept_out,
                         void* workspace, void* stream);

/* msd_sample_token without a workspace argument: the scratch lives in a static device array
 * of the library (one per device, 1,326,336 bytes, held until the process ends; sized for the
 * largest vocabulary, so vocab <= 32768 and MSD_E_CONFIG beyond).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  It calls no allocating
 * routine.  All calls on one device share the scratch, so calls that overlap on one device
 * (two streams, two threads) race; calls ordered on one stream are safe.  The scratch needs
 * no initialisation and each call overwrites what it reads.  Same arguments, numerics and
 * errors as msd_sample_token otherwise. */
int32_t msd_sample_token_noalloc(const float* logits, int32_t vocab, double temperature, double top_p,
                                 double rep_penalty, uint8_t* seen, const double* uniform,
                                 int32_t* token_out, float* probs_out, int32_t* kept_out, void* stream);

/* Bytes of device workspace msd_prefill needs for a prompt of n_tokens tokens. */
int64_t msd_prefill_workspace_bytes(const msd_config* cfg, int32_t n_tokens);

/* Bytes of the tile copy of the layer weights (the QKV, O, gate/up and down matrices and the two
 * RMSNorm scales of every layer: the same bf16 values as packed_w's, 2 bytes each). */
int64_t msd_tiles_bytes(const msd_config* cfg);

/* Writes the tile copy of packed_w's projection matrices to `tiles` (msd_tiles_bytes bytes,
 * 16-byte aligned, device memory): every N x K matrix as 16-row x 32-column tiles of 1 KB in
 * matrix-core operand order (lane l of tile (n / 16, k / 32) holds row 16 (n / 16) + l % 16,
 * columns 32 (k / 32) + 8 (l / 16) .. + 8), tile (n / 16, k / 32) at ((n / 16) (K / 32) +
 * k / 32) * 512 elements, layer after layer, each layer followed by its two RMSNorm scales in
 * packed order.  The O and down rows are in packed order, the gate/up row pairs in the down
 * projection's input order and the O columns in natural order, so the passes' epilogues write
 * contiguous runs.  The multi-row passes (msd_prefill, msd_prefill_paged,
 * msd_verify and the multi-kernel pass of msd_batch_decode_step) read their projection weights
 * from it when it is given: a fragment load is then one 1 KB piece instead of 16 row segments
 * (with the fused epilogues and folded norms it allows, 128-token prefill of the 306M model
 * measured 1.79 -> 1.02 ms).  Rebuild it whenever packed_w changes. */
int32_t msd_pack_tiles(const msd_config* cfg, const void* packed_w, void* tiles, void* stream);

/* Forward pass over a prompt: tokens[0..n_tokens) at positions 0..n_tokens-1 (device int32).
 * Writes the KV cache rows 0..n_tokens-1 of every layer (bf16, post-RoPE K) and the f32
 * logits of the last position; with logits_all != NULL also the logits of every position
 * (n_tokens x vocab_size, row-major).  next_token (device int32[2]) receives the argmax of the
 * last position's logits (lowest index on ties) and a status word (bit 1 = a token id was out
 * of range).  Every projection runs on the matrix cores with its f32 input split into two bf16
 * parts (hi = bf16(x), lo = bf16(x - hi): x to about 2^-17 relative) against the bf16 weights,
 * accumulated in f32; residual stream, RoPE, softmax and SwiGLU are f32 (model.py's maths).
 * Weight arguments as for msd_decode_step; `tiles` is the tile copy of packed_w (msd_pack_tiles)
 * or NULL (the projections then read packed_w's rows: same results, slower).  Requires d_model,
 * 2*d_ff and vocab_size to be multiples of 64, d_ff a multiple of 32 and n_tokens <= context_len. */
int32_t msd_prefill(const msd_config* cfg, const void* token_emb, const void* output_proj,
                    const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                    const int32_t* tokens, int32_t n_tokens, void* kv, void* workspace,
                    float* logits_last, float* logits_all, int32_t* next_token, void* stream);

/* Launch mode of the multi-row passes (msd_prefill, msd_prefill_paged, msd_verify and the
 * multi-kernel pass of msd_batch_decode_step).  With graphs on (off by default; the environment
 * variable MSD_LAUNCH_GRAPHS=1 starts with them on) the ~130 dependent launches of a pass are
 * captured once per argument set (shape, device pointers, sizes) into a HIP graph that is kept
 * (at most 16 per process, the least recently used dropped) and replayed on the caller's stream.
 * That cuts the host's enqueue time per pass from ~0.35 to ~0.07 ms (306M) but runs ~1 % slower
 * on the device, so it is for callers whose host thread is the bottleneck.  Buffer contents are
 * read when the kernels run, so a pass over new tokens in the same buffers replays the same
 * graph.  A stream the caller is capturing gets the launches directly.  Results are bitwise the
 * same either way.  Returns the previous setting.  No counterpart in the reference: a
 * launch-mode switch of this library. */
int32_t msd_set_launch_graphs(int32_t enabled);

/* Bytes of device workspace msd_verify needs for n_tokens rows. */
int64_t msd_verify_workspace_bytes(const msd_config* cfg, int32_t n_tokens);

/* Speculative-decode verification: the target model's forward pass over tokens[0..n_tokens)
 * (device int32) at positions start_pos..start_pos+n_tokens-1, over a contiguous KV cache that
 * holds rows 0..start_pos-1.  Row i attends as a decode step at its position: cached rows
 * 0..start_pos+i-1 as stored (bf16; the rows of tokens 0..i-1 are written by this call first)
 * and its own un-rounded K/V (multi_sm_decode.py:182-221), so its logits are those the
 * sequential decode steps would give once tokens 0..i-1 are accepted.  Writes the K/V rows of
 * every position, the f32 logits of every row (n_tokens x vocab_size) and argmax[2i] = the
 * argmax of row i (lowest index on ties), argmax[2i+1] = status (bit 1 = a token id out of
 * range).  Numerics of msd_prefill (projection inputs as hi/lo bf16 parts); `tiles` as there.
 * Requires start_pos >= 1, start_pos + n_tokens <= context_len <= 512.
 * Replaces the parallel verification kernel the reference describes (K draft tokens through the
 * full target in one call, a mini-prefill with an existing KV cache: knowledge/program.md:
 * 147-155; no code of it is in the reference snapshot, so the interface is this library's own). */
int32_t msd_verify(const msd_config* cfg, const void* token_emb, const void* output_proj,
                   const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                   const int32_t* tokens, int32_t n_tokens, int32_t start_pos, void* kv, void* workspace,
                   float* logits, int32_t* argmax, void* stream);

/* Paged KV cache (used by msd_prefill_paged and msd_batch_decode_step): a pool of pages of 16
 * positions, bf16, laid out [layer][K, V][kv_head][pool_pages * 16][d_head].  A sequence's
 * position p is stored at page page_table[p / 16], slot p % 16.  (The contiguous cache of
 * msd_decode_step is the pool of context_len / 16 pages with the identity table.)
 * Entries outside [0, pool_pages) and positions outside [0, context_len) or past a table are
 * replaced by 0 and reported in the status word (bit 2); the call itself never leaves the pool. */

/* msd_prefill into a paged cache: page_table is a device int32 array of max_pages entries
 * (max_pages * 16 >= n_tokens, max_pages <= ceil(context_len / 16)) for this sequence. */
int32_t msd_prefill_paged(const msd_config* cfg, const void* token_emb, const void* output_proj,
                          const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                          const int32_t* tokens, int32_t n_tokens, const int32_t* page_table,
                          int32_t max_pages, void* kv_pool, int32_t pool_pages, void* workspace,
                          float* logits_last, int32_t* next_token, void* stream);

/* Bytes of device workspace msd_batch_decode_step needs for `batch` sequences.  The workspace
 * must be zero-filled before its first step and then kept for the steps of this batch decoder
 * (it holds the persistent step's epoch and barrier flags); one step may be in flight per
 * workspace.  Any device memory works; for the persistent step (batch <= 8 on a config with
 * MSD_PATH_BATCHED_STEP) uncached memory from msd_workspace_acquire makes its barrier polls
 * cheaper (306M, 8 sequences: 0.786 -> 0.758 ms per step), while the multi-kernel pass of
 * larger batches wants ordinary (cached) memory. */
int64_t msd_batch_workspace_bytes(const msd_config* cfg, int32_t batch);

/* One decode step of `batch` independent sequences: sequence b feeds tokens[b] at position
 * positions[b] (device int32 arrays), reads its cached rows 0..positions[b]-1 through
 * page_tables[b * max_pages ...] and writes its K/V row at positions[b].  Outputs logits
 * (batch x vocab_size f32) and next_tokens (device int32[2 * batch]: argmax of row b at 2b,
 * the step's status word at 2b+1; bit 1 = token out of range, bit 2 = position or page out of
 * range, bit 0 = a wait of the persistent step timed out).  Same numerics as msd_prefill
 * (projection inputs as hi/lo bf16 parts); the
 * current position attends with its un-rounded K/V.  Up to 8 sequences run as ONE persistent
 * launch (one workgroup per compute unit, all resident, grid barriers between the phases of a
 * layer); larger batches, or a device that cannot hold the grid resident, take the multi-kernel
 * matrix-core pass, which reads `tiles` (as for msd_prefill; NULL allowed). */
int32_t msd_batch_decode_step(const msd_config* cfg, const void* token_emb, const void* output_proj,
                              const void* packed_w, const void* tiles, const void* lnf_s, const float* rope,
                              const int32_t* tokens, const int32_t* positions, int32_t batch,
                              const int32_t* page_tables, int32_t max_pages, void* kv_pool,
                              int32_t pool_pages, void* workspace, float* logits,
                              int32_t* next_tokens, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSDECODE_H */
