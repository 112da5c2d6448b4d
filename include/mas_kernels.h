/*
 * mas_kernels.h - C ABI of the MI355X (gfx950) per-layer kernels of mini-agent-serve's
 * Devstral/Mistral decoder: fused residual-add + RMSNorm (bf16 and fp8-e4m3fn outputs),
 * SiluAndMul, NeoX / GPT-J rotary embedding from a cos/sin table, the paged KV-cache append
 * (block-table and slot-mapping forms) and the token-embedding gather.
 *
 * Also: SiluAndMul fused with the fp8 quantize of the down_proj input, RoPE + paged KV append
 * (+ llama-4 query scale) in one kernel, the step's sample placeholders resolved with the
 * embedding gather, and paged attention over the KV cache: split-KV decode and causal context
 * (prefill), each optionally writing the o_proj input's fp8 quantize.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers; tensors are bf16 unless stated (bf16 travels as raw 16-bit
 *     words, fp8 as raw bytes). Strides are in ELEMENTS of the pointed-to type, and the last
 *     (hidden / head_dim) dimension is always contiguous.
 *   - Work is enqueued on `stream` and nothing else: no allocation, no host synchronisation,
 *     no use of the null stream, so every call may be captured into a HIP graph.
 *   - The return value is MAS_OK (0), a negative MAS_ERR_* argument error (nothing was
 *     enqueued), or a positive hipError_t reported by the launch.
 *   - Index inputs are range-checked on the device. A row whose index is out of range is left
 *     unwritten (embedding: zero-filled) and, when `err` is non-NULL, the kernel ORs a
 *     MAS_ERRBIT_* bit into *err. No kernel reads or writes outside the buffers described.
 *
 * Reference interfaces replaced (paths relative to the mini-agent-serve repository):
 *   miniagentserve/models/devstral2/devstral2.py:18-23  flashinfer imports (norm, activation, rope,
 *                                                       page, decode and prefill attention)
 *   miniagentserve/models/devstral2/devstral2.py:260,282 nn.Embedding
 *   miniagentserve/engine/model_runner.py:149-154        ModelRunner.fill_placeholders
 */
#ifndef MAS_KERNELS_H
#define MAS_KERNELS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MAS_OK 0
#define MAS_ERR_INVALID_VALUE (-1) /* null pointer, negative size, bad stride or eps       */
#define MAS_ERR_UNSUPPORTED (-2)   /* a shape this library does not implement             */
#define MAS_ERR_MISALIGNED (-3)    /* a pointer or stride breaks the kernel's alignment   */
#define MAS_ERR_DEVICE (-4)        /* hipGetDevice / device-attribute query failed        */
#define MAS_ERR_SCRATCH (-5)       /* the call needs more scratch than the no-allocation
                                      entry point's static buffer holds                    */
#define MAS_ERR_NOT_READY (-6)     /* the no-allocation entry point's first call on a device
                                      came under graph capture: make one call outside it   */

#define MAS_ERRBIT_TOKEN_ID 1u  /* embedding: id < 0 or id >= vocab                       */
#define MAS_ERRBIT_POSITION 2u  /* rope: position < 0 or >= table rows; kv: position < 0;
                                   attention: seq_len out of range, or (context) a row with
                                   more query tokens than max_q_len                         */
#define MAS_ERRBIT_BATCH 4u     /* kv: batch index outside [0, batch)                     */
#define MAS_ERRBIT_PAGE 8u      /* kv: page slot past kv_indices or page id out of range  */
#define MAS_ERRBIT_SLOT 16u     /* kv slot form: slot >= num_pages * page_size            */
#define MAS_ERRBIT_PLACEHOLDER 32u /* embedding: placeholder -1 - r with r >= num_last     */

/* Library version, (major << 16) | (minor << 8) | patch. */
int mas_version(void);

/* Human-readable text for a return code of this library. */
const char* mas_status_string(int status);

/*
 * Fused residual add + RMSNorm, bf16 output written in place over `input`:
 *   s = f32(input) + f32(residual);  residual <- bf16(s);
 *   input <- bf16(s * rsqrt(mean(s*s) + eps) * f32(weight))
 * input/residual: [rows, hidden]; weight: [hidden].
 * Replaces flashinfer.norm.fused_add_rmsnorm(input, residual, weight, eps, enable_pdl)
 * called at miniagentserve/models/devstral2/devstral2.py:305-307.
 */
int mas_fused_add_rmsnorm_bf16(void* input, int64_t input_stride, void* residual, int64_t residual_stride,
                               const void* weight, int64_t rows, int64_t hidden, float eps,
                               hipStream_t stream);

/*
 * Fused residual add + RMSNorm with a per-tensor fp8 (OCP e4m3fn) output; `input` is read only:
 *   s as above;  residual <- bf16(s);
 *   out <- e4m3fn(clamp(s * rsqrt(mean(s*s) + eps) * f32(weight) / scale, -448, 448))
 * `scale` is read from the device word `scale_dev` when it is non-NULL, else `scale_host` is used.
 * NaN stays NaN (code 0x7f with the input's sign). out: [rows, hidden] bytes.
 * Replaces flashinfer.norm.fused_add_rmsnorm_quant(out, input, residual, weight, scale, eps,
 * enable_pdl) called at miniagentserve/models/devstral2/devstral2.py:241-252.
 */
int mas_fused_add_rmsnorm_quant_fp8(void* out, int64_t out_stride, const void* input, int64_t input_stride,
                                    void* residual, int64_t residual_stride, const void* weight,
                                    const float* scale_dev, float scale_host, int64_t rows, int64_t hidden,
                                    float eps, hipStream_t stream);

/*
 * SiluAndMul gating: out[r, i] = bf16(silu(f32(in[r, i])) * f32(in[r, inter + i])), i < inter
 * (gate half first, up half second). in: [rows, 2*inter]; out: [rows, inter].
 * Replaces flashinfer.activation.silu_and_mul(input, enable_pdl) called at
 * miniagentserve/models/devstral2/devstral2.py:224.
 */
int mas_silu_and_mul_bf16(void* out, int64_t out_stride, const void* input, int64_t input_stride,
                          int64_t rows, int64_t inter, hipStream_t stream);

/*
 * SiluAndMul with the per-tensor fp8 quantize of its result fused in:
 *   y = bf16(silu(f32(in[r, i])) * f32(in[r, inter + i]))            (the unfused op's output)
 *   out[r, i] = e4m3fn(clamp(f32(y) / scale, -448, 448))             (NaN stays NaN)
 * `scale` is read from `scale_dev` when it is non-NULL, else `scale_host` is used. out: bytes.
 * Replaces the silu_and_mul call at miniagentserve/models/devstral2/devstral2.py:224 together with
 * the quantize_fp8 that down_proj applies to its result (devstral2.py:93-95,110-111).
 */
int mas_silu_and_mul_quant_fp8(void* out, int64_t out_stride, const void* input, int64_t input_stride,
                               int64_t rows, int64_t inter, const float* scale_dev, float scale_host,
                               hipStream_t stream);

/*
 * Rotary embedding in place from a cos/sin table, applied to q and k heads.
 * q: rows x num_q_heads heads; head h of row t starts at q + t*q_stride + h*q_head_stride
 * (k likewise). table: fp32 [table_rows, rotary_dim] with row stride `table_stride`; the first
 * rotary_dim/2 columns are cos, the rest sin. The first `rotary_dim` elements of each head are
 * rotated; the remaining head_dim - rotary_dim are untouched.
 *   is_neox != 0: pairs (i, i + rotary_dim/2) use cos[i], sin[i]   (rotate-half)
 *   is_neox == 0: pairs (2i, 2i + 1)          use cos[i], sin[i]   (interleaved)
 *   x_a' = x_a*cos - x_b*sin;  x_b' = x_b*cos + x_a*sin   (fp32 math, one bf16 rounding)
 * positions: `rows` indices, int32 when pos_is_int64 == 0, else int64.
 * rotary_dim must be one of 32, 64, 128, 256, 512 and <= head_dim.
 * Replaces flashinfer.rope.apply_rope_with_cos_sin_cache_inplace(positions, query, key,
 * head_size, cos_sin_cache, is_neox) called at miniagentserve/models/devstral2/devstral2.py:163-166.
 */
int mas_rope_cos_sin_cache_bf16(void* q, int64_t q_stride, int64_t q_head_stride, int64_t num_q_heads,
                                void* k, int64_t k_stride, int64_t k_head_stride, int64_t num_k_heads,
                                const void* positions, int pos_is_int64, const float* table,
                                int64_t table_stride, int64_t table_rows, int64_t rows, int64_t head_dim,
                                int64_t rotary_dim, int is_neox, uint32_t* err, hipStream_t stream);

/*
 * Paged KV-cache append, block-table form. For token t:
 *   b = batch_indices[t], p = positions[t],
 *   page = kv_indices[kv_indptr[b] + p / page_size], entry = p % page_size,
 *   k_cache[page, entry, h, :] = key[t, h, :]  and the same for value, for h < num_heads.
 * Cache element (page, entry, h, d) is at cache + page*page_stride + entry*entry_stride +
 * h*head_stride + d, which covers the NHD ([pages, page_size, heads, dim]) and HND
 * ([pages, heads, page_size, dim]) layouts. key/value element (t, h, d) is at
 * key + t*key_stride + h*key_head_stride + d. batch_indices, positions, kv_indices and kv_indptr
 * are int32; `batch` = number of kv_indptr entries - 1, `num_indices` = kv_indices length.
 * Duplicate destinations are allowed (one of the writers wins).
 * Replaces flashinfer.page.append_paged_kv_cache(append_key, append_value, batch_indices,
 * positions, paged_kv_cache, kv_indices, kv_indptr, kv_last_page_len, kv_layout) called at
 * miniagentserve/models/devstral2/devstral2.py:170-173 (kv_last_page_len carries no information
 * the store needs and is not an argument here).
 */
int mas_append_paged_kv_cache_bf16(void* k_cache, void* v_cache, int64_t page_stride, int64_t entry_stride,
                                   int64_t head_stride, int64_t num_pages, int64_t page_size,
                                   const void* key, int64_t key_stride, int64_t key_head_stride,
                                   const void* value, int64_t value_stride, int64_t value_head_stride,
                                   const int32_t* batch_indices, const int32_t* positions,
                                   const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_indptr,
                                   int64_t batch, int64_t rows, int64_t num_heads, int64_t head_dim,
                                   uint32_t* err, hipStream_t stream);

/*
 * Paged KV-cache store, slot-mapping form: slot = slot_mapping[t] (int64), page = slot / page_size,
 * entry = slot % page_size, then as above. A negative slot marks a padding token and is skipped.
 * Equivalent to the block-table form with slot = block_tables[b, p / page_size]*page_size +
 * p % page_size (miniagentserve/models/devstral2/devstral2.py:170-173,289).
 */
int mas_store_kv_slots_bf16(void* k_cache, void* v_cache, int64_t page_stride, int64_t entry_stride,
                            int64_t head_stride, int64_t num_pages, int64_t page_size, const void* key,
                            int64_t key_stride, int64_t key_head_stride, const void* value,
                            int64_t value_stride, int64_t value_head_stride, const int64_t* slot_mapping,
                            int64_t rows, int64_t num_heads, int64_t head_dim, uint32_t* err,
                            hipStream_t stream);

/*
 * RoPE and the paged KV append fused into one pass over the token rows: q and k are rotated in
 * place exactly as by mas_rope_cos_sin_cache_bf16 (rotary_dim = head_dim, int32 positions), and
 * the rotated k plus v are written to the cache exactly as by mas_append_paged_kv_cache_bf16 with
 * the same positions. Each k row is read once and one kernel is launched instead of two. A
 * position outside the table skips the rotation of that token (its unrotated k is stored); a
 * destination out of range skips its cache write; both are reported through `err` as above.
 * head_dim must be one of 32, 64, 128, 256, 512; table_rows must be at least 1 when there are
 * rows and heads (each token's table row is loaded before its position is judged).
 * Optional llama-4 query scaling: when q_scale_table (bf16, q_scale_rows entries, row k =
 * bf16(1 + beta * log1p(k))) is given, q ends as bf16(f32(bf16(rope(q))) *
 * f32(q_scale_table[pos / q_scale_interval])), the reference's query_states after its two-rounding
 * multiply; a position past the table leaves q rotated, unscaled and reported (POSITION bit).
 * Pass NULL (rows and interval then ignored) for no scaling.
 * Replaces the call sequence at miniagentserve/models/devstral2/devstral2.py:163-179
 * (apply_rope_with_cos_sin_cache_inplace, append_paged_kv_cache on the same rows, then the
 * llama-4 query scale).
 */
int mas_rope_append_paged_kv_cache_bf16(void* q, int64_t q_stride, int64_t q_head_stride, int64_t num_q_heads,
                                        void* k, int64_t k_stride, int64_t k_head_stride, const void* v,
                                        int64_t v_stride, int64_t v_head_stride, int64_t num_kv_heads,
                                        const int32_t* positions, const float* table, int64_t table_stride,
                                        int64_t table_rows, int64_t rows, int64_t head_dim, int is_neox,
                                        void* k_cache, void* v_cache, int64_t page_stride, int64_t entry_stride,
                                        int64_t head_stride, int64_t num_pages, int64_t page_size,
                                        const int32_t* batch_indices, const int32_t* kv_indices,
                                        int64_t num_indices, const int32_t* kv_indptr, int64_t batch,
                                        const void* q_scale_table, int64_t q_scale_rows, int64_t q_scale_interval,
                                        uint32_t* err,
                                        hipStream_t stream);

/*
 * Token-embedding gather: out[t, :] = weight[ids[t], :], a bit copy. ids: int64 [rows];
 * weight: [vocab, hidden] with row stride weight_stride; out: [rows, hidden].
 * Replaces nn.Embedding.forward at miniagentserve/models/devstral2/devstral2.py:260,282.
 */
int mas_embedding_bf16(void* out, int64_t out_stride, const void* weight, int64_t weight_stride, int64_t vocab,
                       const int64_t* ids, int64_t rows, int64_t hidden, uint32_t* err, hipStream_t stream);

/*
 * The step-input path: placeholder resolution fused with the gather. An id -1 - r in ids stands
 * for last_tokens[r] (int32 [num_last], the previous step's samples, still on the GPU); each is
 * replaced in ids by that sample, as fill_placeholders does, and the row of the resolved id is
 * gathered as by mas_embedding_bf16. Non-negative ids are read only. A placeholder with
 * r >= num_last keeps its id, gets a zero row and sets MAS_ERRBIT_PLACEHOLDER. With out == NULL
 * (or hidden == 0) only the ids are resolved: the drop-in for fill_placeholders alone.
 * Replaces ModelRunner.fill_placeholders (miniagentserve/engine/model_runner.py:149-154) and the
 * embed_tokens call that reads its result (miniagentserve/models/devstral2/devstral2.py:282).
 */
int mas_embedding_fill_placeholders_bf16(void* out, int64_t out_stride, const void* weight, int64_t weight_stride,
                                         int64_t vocab, int64_t* ids, int64_t rows, int64_t hidden,
                                         const int32_t* last_tokens, int64_t num_last, uint32_t* err,
                                         hipStream_t stream);

/*
 * Paged decode attention: for each row b and query head h (kv head h / (num_q_heads /
 * num_kv_heads)), over the positions p < seq_lens[b] whose key/value rows sit at
 * page = block_tables[b * block_table_stride + p / page_size], entry = p % page_size:
 *   out[b, h] = bmm2_scale * sum_p softmax_p(bmm1_scale * q[b, h] . k_p) * v_p   (fp32, bf16 out).
 * q, out: [batch, num_q_heads, head_dim] with row / head strides; caches as for the append above
 * (page, entry, head strides); block_tables int32 [batch, max_blocks]; seq_lens int32 [batch].
 * head_dim in {64, 128, 256}; num_q_heads / num_kv_heads <= 16; page_size a power of two.
 * `workspace` (16-byte aligned, workspace_bytes long) holds the per-split partials: a split is
 * chunks_per_split chunks of 256 positions, with chunks_per_split the smallest power of two whose
 * partials fit (mas_paged_decode_attention_workspace_bytes), with at most 64 splits per row and
 * batch * num_kv_heads * splits within 16384 work items (longer splits past those). Grids of fewer
 * such items than the GPU has SIMDs split rows into 128 or 64 positions instead (at most 128 splits
 * per row), when the workspace holds those partials. These lengths bound a row's splits; each row
 * picks its own on the device from its length (256 positions, or 128 / 64 when the rows x kv heads
 * leave 4+ SIMDs per row), so a block table far wider than the rows does not lengthen them. A page id
 * outside [0, num_pages) skips its position (MAS_ERRBIT_PAGE); a seq_len outside
 * [0, max_blocks * page_size] is clamped (MAS_ERRBIT_POSITION); a row with no position gets zeros.
 * With out_fp8, `out` receives e4m3fn codes (strides in elements, as for bf16): the output is
 * rounded to bf16, then quantized as the reference quantizes the o_proj input
 * (devstral2.py:93-95,110-111): e4m3fn(clamp(bf16(O) / scale, -448, 448)), scale read from
 * out_scale_dev (an fp32 device scalar) or, when that is NULL, out_scale_host.
 * Replaces flashinfer.decode.trtllm_batch_decode_with_kv_cache at
 * miniagentserve/models/devstral2/devstral2.py:184-196 (kv_layout "NHD", no sliding window).
 */
int mas_paged_decode_attention_bf16(void* out, int64_t out_stride, int64_t out_head_stride, const void* q,
                                    int64_t q_stride, int64_t q_head_stride, const void* k_cache, const void* v_cache,
                                    int64_t page_stride, int64_t entry_stride, int64_t head_stride, int64_t num_pages,
                                    int64_t page_size, const int32_t* block_tables, int64_t block_table_stride,
                                    int64_t max_blocks, const int32_t* seq_lens, int64_t batch, int64_t num_q_heads,
                                    int64_t num_kv_heads, int64_t head_dim, float bmm1_scale, float bmm2_scale,
                                    int out_fp8, const float* out_scale_dev, float out_scale_host, void* workspace,
                                    int64_t workspace_bytes, uint32_t* err, hipStream_t stream);

/*
 * Paged causal attention of prompt rows (context / chunked prefill): row j owns query tokens
 * [cu_seqlens_q[j], cu_seqlens_q[j + 1]) (q_len) of q and out ([tokens, num_q_heads, head_dim],
 * row / head strides) and seq_lens[j] = kv_len positions in the cache, the last q_len of them its
 * own tokens: token i sits at position kv_len - q_len + i and attends to positions 0..that.
 * For query head h (kv head h / (num_q_heads / num_kv_heads)):
 *   out[t, h] = bmm2_scale * sum_p softmax_p(bmm1_scale * q[t, h] . k_p) * v_p
 * with fp32 accumulation and P rounded to bf16 for the P.V product. max_q_len must bound q_len (it
 * sizes the grid; a longer row's tokens past it are left unwritten, MAS_ERRBIT_POSITION).
 * head_dim 64 or 128; page_size a power of two. A seq_len outside
 * [q_len, max_blocks * page_size] is clamped (MAS_ERRBIT_POSITION; tokens left before position 0
 * get zeros); a page id outside [0, num_pages) skips its position (MAS_ERRBIT_PAGE).
 * out_fp8 / out_scale_dev / out_scale_host: the fp8 output as for mas_paged_decode_attention_bf16.
 * `workspace` (16-byte aligned, workspace_bytes long; NULL / 0 for none; its contents on entry do
 * not matter): when the grid (kv heads x token tiles of max_q_len x rows) has fewer workgroups
 * than the GPU has CUs, each token tile's key range is split over up to 32 workgroups whose
 * partials go here - rows * ceil(max_q_len / tile) * tile * num_q_heads * splits * (head_dim + 2)
 * * 4 bytes, tile = 32 tokens x (workgroup wavefronts / heads per workgroup) - and a second kernel
 * merges them; with less workspace, fewer splits or none. Each token tile divides its own key
 * range among the splits; max_kv_len (<= 0: none; else the block table's reach) is a hint that
 * only sizes the choice of the split count. A grid of 8 or more rows and at most 1024 tokens per
 * row that has a workgroup per CU or more (a captured graph's padded prompt rows, max_q_len the
 * step's tokens) is planned on the device when the workspace holds the plan: a first kernel reads
 * cu_seqlens_q / seq_lens, picks the split count for the real lengths and writes the work items
 * to the workspace (its counts, 32 bytes per workgroup of the grid, 32 per (row, token tile), then
 * the partials), and the merge runs over the split tiles only. Calls sharing a workspace must not
 * overlap.
 * Replaces flashinfer.prefill.trtllm_batch_context_with_kv_cache at
 * miniagentserve/models/devstral2/devstral2.py:198-213 (kv_layout "NHD", no sliding window).
 */
int mas_paged_context_attention_bf16(void* out, int64_t out_stride, int64_t out_head_stride, const void* q,
                                     int64_t q_stride, int64_t q_head_stride, const void* k_cache,
                                     const void* v_cache, int64_t page_stride, int64_t entry_stride,
                                     int64_t head_stride, int64_t num_pages, int64_t page_size,
                                     const int32_t* block_tables, int64_t block_table_stride, int64_t max_blocks,
                                     const int32_t* seq_lens, const int32_t* cu_seqlens_q, int64_t num_rows,
                                     int64_t max_q_len, int64_t max_kv_len, int64_t num_q_heads, int64_t num_kv_heads,
                                     int64_t head_dim, float bmm1_scale, float bmm2_scale, int out_fp8,
                                     const float* out_scale_dev, float out_scale_host, void* workspace,
                                     int64_t workspace_bytes, uint32_t* err, hipStream_t stream);

/*
 * mas_paged_decode_attention_bf16 without a workspace argument: the same kernels and results, with
 * the split partials in a scratch array the library keeps in device memory, one per GPU it runs on,
 * MAS_DECODE_ATTENTION_SCRATCH_BYTES long, held until the process ends. The array is part of the
 * library's code object: every process that loads the library holds it on each GPU where the library's
 * kernels are loaded, whether or not it calls this entry point. No allocation happens in the
 * call: the array's address is looked up once per device, on the first call there (the caller's
 * current device is left as it was). That first call must not be made while `stream` is being
 * captured into a graph (the lookup may load the code object): it then returns MAS_ERR_NOT_READY and
 * enqueues nothing; one call outside capture per device sets the lookup up, after which captured
 * calls work. Splits are made as long as needed for the partials to fit the
 * array; a call that does not fit even with one split per row (batch * num_q_heads * (head_dim + 2)
 * * 4 bytes over the limit) returns MAS_ERR_SCRATCH and enqueues nothing. Every call on one GPU
 * uses that GPU's one array: calls that overlap in time on one GPU (on different streams) race and
 * must be ordered by the caller; consecutive calls on one stream are safe. Nothing in the array
 * needs clearing between calls.
 * No counterpart in the reference (it always passes a workspace, devstral2.py:36-42,187): this is
 * for callers that cannot allocate a workspace - code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.
 */
#define MAS_DECODE_ATTENTION_SCRATCH_BYTES (64ll << 20)
int mas_paged_decode_attention_bf16_noalloc(void* out, int64_t out_stride, int64_t out_head_stride, const void* q,
                                            int64_t q_stride, int64_t q_head_stride, const void* k_cache,
                                            const void* v_cache, int64_t page_stride, int64_t entry_stride,
                                            int64_t head_stride, int64_t num_pages, int64_t page_size,
                                            const int32_t* block_tables, int64_t block_table_stride,
                                            int64_t max_blocks, const int32_t* seq_lens, int64_t batch,
                                            int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                            float bmm1_scale, float bmm2_scale, int out_fp8,
                                            const float* out_scale_dev, float out_scale_host, uint32_t* err,
                                            hipStream_t stream);

/*
 * Workspace bytes mas_paged_decode_attention_bf16 needs when each split covers chunks_per_split
 * chunks of 256 positions (1: the most parallel split). -1 for invalid arguments.
 * No counterpart in the reference (its caller passes a fixed 128 MiB workspace,
 * miniagentserve/models/devstral2/devstral2.py:36-42).
 */
int64_t mas_paged_decode_attention_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim,
                                                   int64_t max_blocks, int64_t page_size, int64_t chunks_per_split);

/*
 * Workspace bytes that let mas_paged_context_attention_bf16 split every small grid of these
 * sizes the most (32 splits per token tile); less gets fewer splits or none. -1 for invalid
 * arguments (num_q_heads not a multiple of num_kv_heads, head_dim not 64 or 128).
 * No counterpart in the reference (its caller passes a fixed 128 MiB workspace,
 * miniagentserve/models/devstral2/devstral2.py:36-42).
 */
int64_t mas_paged_context_attention_workspace_bytes(int64_t num_rows, int64_t max_q_len, int64_t num_q_heads,
                                                    int64_t num_kv_heads, int64_t head_dim);

#ifdef __cplusplus
}
#endif

#endif /* MAS_KERNELS_H */
