/* C ABI of the MI355X (gfx950) HilbertA inference attention path.
 *
 * Plain pointers and sizes only; every device pointer is a HIP device allocation on the
 * current device, every launch is asynchronous on `stream` and never synchronises.
 * Return value: 0 on success, HB_EINVAL (1) for a rejected argument, HB_EHIP (2) for a HIP
 * runtime error; hb_last_error() gives the message (thread-local).
 *
 * Python binds these through ctypes (hilberta_amd/_lib.py); INTEGRATION.md shows the binding
 * the reference package would add.
 */
#ifndef HILBERTA_HIP_H
#define HILBERTA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HB_ABI_VERSION 1
#define HB_DTYPE_BF16 0
#define HB_DTYPE_F16 1

typedef struct ihipStream_t* hb_stream_t;

const char* hb_last_error(void);
int hb_version(void);

/* ---------------------------------------------------------------- (c) block-sparse attention
 * Workspace needed by hb_paired_fwd / hb_block_sparse_fwd for these shapes (bytes, or -1 when
 * the shapes are rejected).  The workspace must start zero-filled once; the kernels leave their
 * counters at zero when they finish, so one workspace serves every later launch on one stream.
 * Launches that overlap in time must not share a workspace.
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
 *   kv_indices, kv_flags : int32 [(N-G)/128, table_width]; kv_counts int32 [(N-G)/128]
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

/* Unpaired-table forward (64-query rows, no flags).  Replaces _block_sparse_fwd[grid](...) of
 * reference hilberta/sparse_kernel.py:315-339 (kernel :28-97); block_size must be 64. */
int hb_block_sparse_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                        const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                        int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                        const int32_t* kv_counts, int32_t table_width, int32_t global_tokens,
                        int32_t block_size, int32_t all_queries, float scale_log2,
                        void* workspace, int64_t workspace_bytes, int32_t num_groups,
                        hb_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HILBERTA_HIP_H */
