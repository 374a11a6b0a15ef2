/* C ABI of the MI355X (gfx950) HilbertA inference attention path.
 *
 * Plain pointers and sizes only; every device pointer is a HIP device allocation on the
 * current device, every launch is asynchronous on `stream` and never synchronises.
 * Return value: 0 on success, HB_EINVAL (1) for a rejected argument, HB_EHIP (2) for a HIP
 * runtime error; hb_last_error() gives the message (thread-local).
 *
 * Python binds these through ctypes (hilberta_amd/_lib.py).
 */
#ifndef HILBERTA_HIP_H
#define HILBERTA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HB_ABI_VERSION 4
#define HB_DTYPE_BF16 0
#define HB_DTYPE_F16 1

typedef struct ihipStream_t* hb_stream_t;

const char* hb_last_error(void);
int hb_version(void);

/* Identifier of the graph capture `stream` is taking part in (hipStreamGetCaptureInfo), or 0 when
 * it is not capturing.  No counterpart in the reference: callers that keep per-stream workspaces
 * use it to give every captured graph a workspace of its own. */
int hb_stream_capture_id(hb_stream_t stream, uint64_t* capture_id);

/* ---------------------------------------------------------------- (c) block-sparse attention
 * Workspace needed by hb_paired_fwd / hb_block_sparse_fwd for these shapes (bytes, or -1 when
 * the shapes are rejected).  It holds the work-queue counters (first 256 bytes) and the partial
 * results of split global query tiles.  It must be zero-filled once before first use; every
 * launch leaves the counters at zero again, so one workspace serves all later launches.
 * Launches that overlap in time must not share a workspace.  paired: 0 = unpaired tables
 * (hb_block_sparse_fwd), 1 = paired (hb_paired_fwd), 2 = quad (hb_quad_fwd).
 */
int64_t hb_attention_workspace_bytes(int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                                     int32_t global_tokens, int32_t table_width,
                                     int32_t key_block_size, int32_t paired, int32_t all_queries);

/* Paired-table forward.  Replaces the Triton launch _paired_fwd[(N/128, B*H)](Q, K, V, O, INDICES,
 * FLAGS, COUNTS, strides..., HEADS, N, D, G, MAX_BLOCKS, BLOCK_N, SCALE_LOG2, ALL_QUERIES, ...)
 * of reference hilberta/paired_kernel.py:181-204 (kernel :18-94).
 *   q, k, v, out : [B, H, N, D] bf16/fp16 views, last dim contiguous, 16-byte aligned base
 *   lse          : optional fp32 [B, H, N] natural-log row logsumexp (NULL to skip)
 *   strides      : 12 element strides: q(b,h,n), k(b,h,n), v(b,h,n), out(b,h,n)
 *   kv_indices, kv_flags : int32 [ceil((N-G)/128), table_width]; kv_counts int32 [ceil((N-G)/128)]
 *   N and G     : multiples of 64.  Paired rows are aligned to the end of the sequence: row r
 *                  covers queries N - 128*(rows - r) ..+127, so when N - G is an odd multiple of 64
 *                  row 0's half 0 lies in the global prefix; it is computed but never stored (its
 *                  flags should be 0; hb_pair_rows leaves it empty).  When G is an odd multiple of
 *                  64 the last 128-query global tile reaches 64 queries past G; they are computed
 *                  but never stored either.  (The reference requires N and G multiples of 128.)
 *   key_block_size : 64 or 128 (flag bit half + 2*key_half)
 *   all_queries  : 1 = global query rows attend every key block in this launch
 *                  (the reference's "triton" strategy); 0 = leave global rows untouched
 *   scale_log2   : softmax scale * log2(e)
 *   num_groups   : persistent workgroups (0 = 2 per compute unit)
 */
int hb_paired_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                  const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                  int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                  const int32_t* kv_flags, const int32_t* kv_counts, int32_t table_width,
                  int32_t global_tokens, int32_t key_block_size, int32_t all_queries,
                  float scale_log2, void* workspace, int64_t workspace_bytes, int32_t num_groups,
                  hb_stream_t stream);

/* Quad-table forward: the same launch as hb_paired_fwd (replacing the same reference launch,
 * hilberta/paired_kernel.py:181-204, kernel :18-94) over quad tables, in which paired rows 2r
 * and 2r + 1 are merged into one 256-query row r (hb_quad_rows): kv_indices, kv_flags int32
 * [(N-G)/256, table_width], kv_counts int32 [(N-G)/256], flag bit b (0..3) set where 64-query
 * block b of the row sees the 64-key block.  One eight-wave workgroup per compute unit stages
 * each K/V block once for all 256 queries.  head_dim 128 only; N and G multiples of 256.  Every
 * query sees the same key blocks in the same order with the same arithmetic as under
 * hb_paired_fwd (blocks another query block needs are computed and masked to exact zeros), so
 * ordinary rows are bitwise equal to hb_paired_fwd's; global rows may split into chunks at other
 * places.  num_groups 0 = one per compute unit.  Workspace: hb_attention_workspace_bytes with
 * paired = 2. */
int hb_quad_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                const int32_t* kv_flags, const int32_t* kv_counts, int32_t table_width,
                int32_t global_tokens, int32_t all_queries, float scale_log2, void* workspace,
                int64_t workspace_bytes, int32_t num_groups, hb_stream_t stream);

/* Paired-table forward that allocates nothing.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory or pass a workspace (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments, checks and results as
 * hb_paired_fwd, without workspace / workspace_bytes: the work-queue counters and the split
 * partials live in a static device array of HB_NOALLOC_SCRATCH_BYTES per device, which the
 * library holds from its first use on a device until the process ends.  Shapes whose workspace
 * (hb_attention_workspace_bytes) exceeds that size are rejected with HB_EINVAL before any HIP
 * call.  Every call clears the counters with a fill kernel on `stream` (no memset, no
 * allocation, no hipFree).  All calls on one device share the one array: calls that may overlap
 * in time on one device (different streams, or graphs replayed concurrently) race and must be
 * serialised by the caller. */
#define HB_NOALLOC_SCRATCH_BYTES (32ll << 20)
int hb_paired_fwd_noalloc(const void* q, const void* k, const void* v, void* out, float* lse,
                          const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                          int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                          const int32_t* kv_flags, const int32_t* kv_counts,
                          int32_t table_width, int32_t global_tokens, int32_t key_block_size,
                          int32_t all_queries, float scale_log2, int32_t num_groups,
                          hb_stream_t stream);

/* Unpaired-table forward (64-query rows, no flags).  Replaces _block_sparse_fwd[grid](...) of
 * reference hilberta/sparse_kernel.py:315-339 (kernel :28-97); block_size must be 64. */
int hb_block_sparse_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                        const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                        int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                        const int32_t* kv_counts, int32_t table_width, int32_t global_tokens,
                        int32_t block_size, int32_t all_queries, float scale_log2,
                        void* workspace, int64_t workspace_bytes, int32_t num_groups,
                        hb_stream_t stream);

/* ---------------------------------------------------------------- (a) Hilbert permutation
 * dst[o, i, :] = src[o, index[i], :] for o < outer, i < rows, each row row_bytes contiguous bytes
 * (strides in bytes).  Replaces x.index_select(dim, order) of reference
 * hilberta/flux_adapter.py:209-212 (entry), :243 (exit) and sampling_layout.py:96-97, :110.
 * Indices outside [0, src_rows) are skipped and set *error (device int, may be NULL) to 1. */
int hb_gather_rows(const void* src, void* dst, const int64_t* index, int64_t rows, int64_t outer,
                   int64_t src_outer_stride, int64_t dst_outer_stride, int64_t src_row_stride,
                   int64_t dst_row_stride, int64_t row_bytes, int64_t src_rows, int32_t* error,
                   hb_stream_t stream);

/* ---------------------------------------------------------------- FLUX attention inputs
 * Per-head RMSNorm + rotary embedding + [text; image] concatenation into one BNHD tensor
 * out[b, t, h, :] (head_dim 128).  Replaces, at reference hilberta/flux_adapter.py:283-295,
 * attn.norm_q/norm_k/norm_added_q/norm_added_k (diffusers 0.36.0 RMSNorm), the torch.cat of text
 * and image tokens and apply_rotary_emb (use_real, interleaved pairs).  Tokens t < text_tokens
 * are read from src_text row t, the others from src_image row t - text_tokens (element strides;
 * rows hold heads*128 elements per plane).  planes = 2 prepares Q and K in one launch: plane p is
 * read at column offset p * src_plane_stride and written at p * out_plane_stride.  weights is
 * NULL or a host array of 2*planes device pointers {plane0 text, plane0 image, plane1 text,
 * plane1 image} (entries may be NULL: no weight multiply).  normalize=0 skips the RMSNorm
 * (weights must then be NULL); cos = sin = NULL skips the rotation; cos/sin are fp32
 * [tokens, 128] rows in output token order.  All device pointers 16-byte aligned, strides
 * multiples of 8.  The output must not overlap a source. */
int hb_qk_prep(const void* src_text, const void* src_image, int64_t text_batch_stride,
               int64_t text_row_stride, int64_t image_batch_stride, int64_t image_row_stride,
               int32_t planes, int64_t src_plane_stride, int32_t batch, int32_t text_tokens,
               int32_t tokens, int32_t heads, int32_t head_dim, int32_t dtype, int32_t normalize,
               const void* const* weights, float eps, const float* cos, const float* sin,
               void* out, int64_t out_plane_stride, int64_t out_batch_stride,
               int64_t out_row_stride, hb_stream_t stream);

/* Gated residual update + AdaLN modulation, one pass per row (FLUX blocks).  For each of
 * batch x rows rows of `hidden` values (row i of batch b at base + b*batch_stride + i*row_stride):
 *   r = x + gate[b] * y            (skipped when y is NULL: r = x)
 *   x_out = r                       (when x_out is not NULL; may be x itself)
 *   out = shift[b] + LayerNorm(r) * (1 + scale[b])   (no affine, eps; fp32 statistics)
 * with the 16-bit roundings of the torch sequence (r, the normalised row and 1 + scale are each
 * rounded).  gate is [batch, hidden] with gate_batch_stride, shift/scale with mod_batch_stride.
 * No counterpart in the
 * reference's own code: it replaces diffusers 0.36.0 AdaLayerNormZero / AdaLayerNormZeroSingle /
 * AdaLayerNormContinuous and the gated residual adds of FluxTransformerBlock and
 * FluxSingleTransformerBlock, the blocks of the transformer hilberta/flux_adapter.py wraps.
 * hidden is 512 * {1, 2, 3, 4, 6, 8}; pointers 16-byte aligned; strides multiples of 8;
 * out must not overlap x or y. */
int hb_adaln_modulate(int32_t batch, int32_t rows, int32_t hidden, int32_t dtype, float eps,
                      const void* x, int64_t x_batch_stride, int64_t x_row_stride, const void* y,
                      int64_t y_batch_stride, int64_t y_row_stride, const void* gate,
                      int64_t gate_batch_stride, void* x_out,
                      int64_t x_out_batch_stride, int64_t x_out_row_stride, const void* shift,
                      const void* scale, int64_t mod_batch_stride, void* out,
                      int64_t out_batch_stride, int64_t out_row_stride, hb_stream_t stream);

/* ---------------------------------------------------------------- (b) block tables
 * Hilbert order of a grid_size x grid_size raster (reference hilberta/geometry.py:6-25). */
int hb_hilbert_order(int32_t grid_size, int64_t* out, hb_stream_t stream);

/* Composite order and physical packing (reference hilberta/plan.py:133-150, :186-197):
 * original_order / inverse_original [n], image_order / inverse_image_order [n],
 * physical_original_blocks [nb] (shared blocks first) and original_to_physical [nb] (+ text
 * blocks).  status (device int32[3]) receives {#shared blocks, partial-shared-block flag,
 * 1 if image_order is not a permutation of the image tokens (else 0)}. */
int hb_plan_layout(int32_t grid_size, int32_t block_size, int32_t text_tokens, int32_t shared,
                   int64_t* original_order, int64_t* inverse_original, int64_t* image_order,
                   int64_t* inverse_image_order, int64_t* physical_original_blocks,
                   int64_t* original_to_physical, int32_t* status, hb_stream_t stream);

/* Scratch bytes for the bridge score matrix of one phase (nb * nb int32). */
int64_t hb_plan_scratch_bytes(int32_t grid_size, int32_t block_size);

/* Adjacency bitmap of one phase: bits [ordinary rows][ceil(T/32)] uint32.  Rows hold the global
 * prefix and the same-tile ordinary blocks (plan.py:153-184); bridge_mode 1 adds the directed
 * top-1 bridge of build_plan (plan.py:159-172), 2 the reciprocal top-K of bridge_k_plan
 * (bridge_k.py:21-44).  bridge_original_blocks [nb, k] int64 receives the chosen key blocks
 * (-1 = none); scores is nb*nb int32 scratch. */
int hb_plan_phase_bits(const int64_t* inverse_original, const int64_t* physical_original_blocks,
                       const int64_t* original_to_physical, int32_t grid_size, int32_t tile_count,
                       int32_t text_tokens, int32_t block_size, int32_t shared_blocks,
                       int32_t phase, int32_t bridge_mode, int32_t k, int32_t* scores,
                       int64_t* bridge_original_blocks, uint32_t* bits, hb_stream_t stream);

/* Bitmap of existing unpaired tables (rows x width ids with counts), for pairing them. */
int hb_table_bits(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows, int32_t width,
                  int32_t total_blocks, uint32_t* bits, hb_stream_t stream);

/* Row lengths of a bitmap: unpaired counts [rows] and/or paired counts [rows/2] at
 * key_block_size 64 or 128; max_counts (device int32[2]) receives the widest of each. */
int hb_bits_counts(const uint32_t* bits, int32_t rows, int32_t total_blocks,
                   int32_t key_block_size, int32_t* counts, int32_t* paired_counts,
                   int32_t* max_counts, hb_stream_t stream);

/* Ascending, zero-padded tables from a bitmap: unpaired ids [rows, width] and/or paired ids and
 * flags [rows/2, paired_width] with flag bit (half + 2*key_half) (paired_metadata.py:38-51). */
int hb_bits_emit(const uint32_t* bits, int32_t rows, int32_t total_blocks, int32_t key_block_size,
                 int32_t* ids, int32_t width, int32_t* paired_ids, int32_t* paired_flags,
                 int32_t paired_width, hb_stream_t stream);

/* Pairs an unpaired table in one launch, replacing pair_metadata (paired_metadata.py:26-51) on the
 * device: rows 2r and 2r + 1 of kv_indices [rows, width] (with kv_counts) become paired row r of
 * paired_ids / paired_flags [(rows+1)/2, paired_width], ascending, flag bit (half + 2*key_half),
 * zero-padded, and paired_counts [(rows+1)/2].  An odd row count is paired from the end: paired
 * row r then holds rows 2r - 1 and 2r, and paired row 0 has an empty half 0 (the layout
 * hb_paired_fwd expects for ordinary query counts that are odd multiples of 64; pair_metadata
 * itself rejects odd counts).  paired_width should bound every paired row's entries
 * (min(2*width, key blocks) always does): a longer row is cut to paired_width entries and sets
 * *overflow (device int32, may be NULL; never cleared here) to 1.  total_blocks <= 16384.  No host
 * synchronisation. */
int hb_pair_rows(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows, int32_t width,
                 int32_t total_blocks, int32_t key_block_size, int32_t* paired_ids,
                 int32_t* paired_flags, int32_t* paired_counts, int32_t paired_width,
                 int32_t* overflow, hb_stream_t stream);

/* Fused device plan: bridge_k_plan(tiles, K, shared, grid_size) + pair_metadata for all four
 * phases (reference hilberta/bridge_k.py:10-51, plan.py:133-197, paired_metadata.py:26-51), in
 * two calls with one host read between them.  hb_paired_plan_tables fills the layout (int64 [n]
 * orders, int64 [n/64] block maps, as hb_plan_layout) and, in `scratch`
 * (hb_paired_plan_scratch_bytes), the four phases' adjacency bitmaps, and writes status (device
 * int32[7]) = {#shared blocks, partial-shared-block flag, 1 if the image order is not a
 * permutation, widest paired row of phases 0..3}.  After reading status the caller allocates
 * each phase's paired tables ([(nb - shared)/2, width]) and calls hb_paired_plan_emit with host
 * arrays of the four device pointers and widths.  64-token blocks; at most 16384 image blocks. */
int64_t hb_paired_plan_scratch_bytes(int32_t grid_size, int32_t text_tokens);
int hb_paired_plan_tables(int32_t grid_size, int32_t tile_count, int32_t k, int32_t text_tokens,
                          int32_t shared, int32_t key_block_size, int64_t* original_order,
                          int64_t* inverse_original, int64_t* image_order,
                          int64_t* inverse_image_order, int64_t* physical_original_blocks,
                          int64_t* original_to_physical, void* scratch, int32_t* status,
                          hb_stream_t stream);
int hb_paired_plan_emit(int32_t grid_size, int32_t text_tokens, int32_t shared_blocks,
                        int32_t key_block_size, const void* scratch, int32_t* const* ids,
                        int32_t* const* flags, int32_t* const* counts, const int32_t* widths,
                        hb_stream_t stream);

/* Quad tables for hb_quad_fwd in one launch.  With kv_flags: kv_indices/kv_flags/kv_counts are
 * paired 64-key tables ([rows, width], rows even; pair_metadata's output, reference
 * hilberta/paired_metadata.py:26-51) and quad row r is the union of paired rows 2r and 2r + 1,
 * flag bit 2j + half from paired row 2r + j.  Without (kv_flags NULL): unpaired 64-query tables
 * (rows a multiple of 4), quad row r the union of rows 4r .. 4r + 3, flag bit j from row 4r + j.
 * Rows come out ascending and zero padded to quad_width, with counts; a longer union is cut to
 * quad_width and sets *overflow (device int, may be NULL) to 1.  total_blocks <= 2048.  No
 * counterpart in the reference: it extends the reference's pairing (paired_metadata.py:38-51)
 * from two query blocks to four for the 256-query kernel. */
int hb_quad_rows(const int32_t* kv_indices, const int32_t* kv_flags, const int32_t* kv_counts,
                 int32_t rows, int32_t width, int32_t total_blocks, int32_t* quad_ids,
                 int32_t* quad_flags, int32_t* quad_counts, int32_t quad_width, int32_t* overflow,
                 hb_stream_t stream);

/* ---------------------------------------------------------------- (b) block tables on the host
 * The table builder on the CPU, for callers that set plans up on a host without a GPU (the
 * reference builds every table there: hilberta/geometry.py:6-25, plan.py:114-197,
 * bridge_k.py:10-51, paired_metadata.py:26-51).  Each takes the arguments of the device entry
 * point of the same name without the _host suffix, minus the stream, as host pointers, with the
 * same checks and error codes, and writes the same values bit for bit; it runs synchronously on
 * the calling thread and makes no HIP call.  The attention launches have no host counterpart. */
int hb_hilbert_order_host(int32_t grid_size, int64_t* out);
int hb_plan_layout_host(int32_t grid_size, int32_t block_size, int32_t text_tokens, int32_t shared,
                        int64_t* original_order, int64_t* inverse_original, int64_t* image_order,
                        int64_t* inverse_image_order, int64_t* physical_original_blocks,
                        int64_t* original_to_physical, int32_t* status);
int hb_plan_phase_bits_host(const int64_t* inverse_original, const int64_t* physical_original_blocks,
                            const int64_t* original_to_physical, int32_t grid_size,
                            int32_t tile_count, int32_t text_tokens, int32_t block_size,
                            int32_t shared_blocks, int32_t phase, int32_t bridge_mode, int32_t k,
                            int32_t* scores, int64_t* bridge_original_blocks, uint32_t* bits);
int hb_table_bits_host(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows,
                       int32_t width, int32_t total_blocks, uint32_t* bits);
int hb_bits_counts_host(const uint32_t* bits, int32_t rows, int32_t total_blocks,
                        int32_t key_block_size, int32_t* counts, int32_t* paired_counts,
                        int32_t* max_counts);
int hb_bits_emit_host(const uint32_t* bits, int32_t rows, int32_t total_blocks,
                      int32_t key_block_size, int32_t* ids, int32_t width, int32_t* paired_ids,
                      int32_t* paired_flags, int32_t paired_width);
int hb_pair_rows_host(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows,
                      int32_t width, int32_t total_blocks, int32_t key_block_size,
                      int32_t* paired_ids, int32_t* paired_flags, int32_t* paired_counts,
                      int32_t paired_width, int32_t* overflow);

/* ---------------------------------------------------------------- measurement
 * Dense bf16 MFMA peak probe: `groups` workgroups (0 = two per compute unit) of four waves, each
 * wave issuing `iterations` x 4 independent v_mfma_f32_32x32x16_bf16 back to back; *flops (host
 * int64) receives the floating-point operations of the launch, to be divided by its event-timed
 * duration.  `sink` is a device float array of groups x 256 entries that the kernel never writes
 * for its fixed operands.  No counterpart in the reference: it measures the ceiling the benchmark
 * states its MFMA utilisation against. */
int hb_mfma_peak_probe(int32_t iterations, int32_t groups, float* sink, int64_t* flops,
                       hb_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HILBERTA_HIP_H */
