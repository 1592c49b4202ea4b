/*
 * sia_attention.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Each entry point replaces one function of the reference engine's attention
 * path (Prathmesh234/simple-inference-autoresearch); the reference interface it
 * stands in for is cited above it as file:line.  The Python package next to
 * this header calls these symbols from its thin PyTorch extension (`_sia_ops`,
 * C++) and keeps the reference's Python signatures; it also opens the library
 * with ctypes for the version, status strings and the tests that call the ABI
 * directly.  Any other FFI (cgo, JNI, N-API) can bind them the same way.
 *
 * Conventions shared by every entry point
 *  - Tensors are passed as `sia_tensor` descriptors: a device pointer, a dtype,
 *    the shape and the strides in ELEMENTS (a torch view maps 1:1).  The last
 *    (head_dim) stride must be 1; other strides may describe any view.
 *  - Nothing here allocates device memory, synchronises, or keeps per-call
 *    state: callers own every buffer.  Split-K decode and prefill need a
 *    caller-provided workspace whose size `sia_decode_workspace_size` /
 *    `sia_prefill_workspace_size` reports.
 *  - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the
 *    null stream), so every entry point may be captured in a HIP graph.
 *    `kv_len` is always read on the device.
 *  - Return value: SIA_OK (0) or a negative `sia_status`; a failing call
 *    enqueues nothing.  `sia_status_string` names the code and
 *    `sia_last_error_message` (per thread) says what was wrong.
 *  - The library targets gfx950 only.
 */
#ifndef SIA_ATTENTION_H
#define SIA_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIA_ABI_VERSION 1
#define SIA_MAX_DIMS 5

typedef enum sia_dtype {
  SIA_F16 = 0,
  SIA_BF16 = 1,
  SIA_F32 = 2,
  SIA_I8 = 3,
  SIA_I32 = 4,
  SIA_I64 = 5,
  SIA_U8 = 6
} sia_dtype;

typedef enum sia_status {
  SIA_OK = 0,
  SIA_ERR_INVALID_ARGUMENT = -1, /* shape / dtype / stride / alignment mismatch */
  SIA_ERR_UNSUPPORTED = -2,      /* valid but not implemented (e.g. head_dim 48) */
  SIA_ERR_WORKSPACE = -3,        /* workspace missing or too small */
  SIA_ERR_LAUNCH = -4,           /* the HIP runtime refused the launch */
  SIA_ERR_DEVICE = -5            /* no device / not a gfx950 device */
} sia_status;

typedef struct sia_tensor {
  void* data;                     /* device pointer */
  int32_t dtype;                  /* sia_dtype */
  int32_t ndim;                   /* 0..SIA_MAX_DIMS */
  int64_t shape[SIA_MAX_DIMS];
  int64_t stride[SIA_MAX_DIMS];   /* in elements */
} sia_tensor;

/* Optional knobs for the decode family; pass NULL for the defaults. */
typedef struct sia_decode_options {
  int32_t tiles_per_split;  /* 0 = automatic; else force this many 16-token tiles per split-K item */
  int32_t reserved0;        /* must be zero */
  void* main_begin_event;   /* optional hipEvent_t (created with timing): stamped with the main decode kernel's start */
  void* main_end_event;     /* optional hipEvent_t: stamped with its end (before the split-K reduction); both through
                               hipExtLaunchKernel, so the interval is the kernel's own execution */
  int64_t reserved[4];      /* must be zero */
} sia_decode_options;

int sia_abi_version(void);
const char* sia_status_string(int status);
const char* sia_last_error_message(void);

/* Bytes of workspace the decode entry points need for split-K partials and
 * their device-side plan, for this batch/head geometry on the current device. */
int sia_decode_workspace_size(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                              int64_t head_dim, size_t* bytes);

/* Replaces attention_flash_decode (kernels/flash_decode_kernel.py:119-160).
 * Every decode entry point takes head_dim 16, 32, 64, 128 or 256.
 * q (B,Hq,1,D) f16|bf16|f32; k,v (B,Hkv,S,D) f16|bf16|f32 (views into the
 * cache); kv_len int32 (1,)|()|(B,) on device; out (B,1,Hq,D) dtype of q,
 * 16-byte aligned rows.  16-bit q and K/V run on the MFMA kernels; a float32
 * q or K/V runs every product in fp32 on the vector ALUs, as the reference's
 * decode kernel does (kernels/flash_decode_kernel.py:85-114).  Every decode
 * entry point accepts an f32 q the same way. */
int sia_attention_flash_decode(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v,
                               const sia_tensor* kv_len, float sm_scale, const sia_tensor* out,
                               void* workspace, size_t workspace_bytes,
                               const sia_decode_options* opts, void* stream);

/* Replaces attention_flash_decode_int8 (kernels/flash_decode_int8_kernel.py:121-167).
 * k_int8,v_int8 (B,Hkv,S,D) int8; k_scale,v_scale (B,Hkv,S) f32|f16. */
int sia_attention_flash_decode_int8(const sia_tensor* q, const sia_tensor* k_int8,
                                    const sia_tensor* v_int8, const sia_tensor* k_scale,
                                    const sia_tensor* v_scale, const sia_tensor* kv_len,
                                    float sm_scale, const sia_tensor* out, void* workspace,
                                    size_t workspace_bytes, const sia_decode_options* opts,
                                    void* stream);

/* Replaces gqa_int8_flash_decode (kernels/paged_flash_decode_int8_gqa_kernel.py:100-124).
 * Same arguments as sia_attention_flash_decode_int8; every kernel of this
 * library already reads each KV head once per GQA group. */
int sia_gqa_int8_flash_decode(const sia_tensor* q, const sia_tensor* k_int8,
                              const sia_tensor* v_int8, const sia_tensor* k_scale,
                              const sia_tensor* v_scale, const sia_tensor* kv_len,
                              float sm_scale, const sia_tensor* out, void* workspace,
                              size_t workspace_bytes, const sia_decode_options* opts,
                              void* stream);

/* Replaces paged_attention_flash_decode (kernels/paged_flash_decode_kernel.py:107-152).
 * k_pool,v_pool (num_pages,Hkv,page_size,D) f16|bf16; block_table (B,max_blocks)
 * int32; page_size any positive size: 16 * 2^k runs on the MFMA kernels, any
 * other size (1, 2, 4, 8, ... as the reference's tl.arange(0, PAGE_SIZE)
 * takes) on the fp32 vector-ALU kernel, which looks up each token's page. */
int sia_paged_attention_flash_decode(const sia_tensor* q, const sia_tensor* k_pool,
                                     const sia_tensor* v_pool, const sia_tensor* block_table,
                                     const sia_tensor* kv_len, int32_t page_size, float sm_scale,
                                     const sia_tensor* out, void* workspace,
                                     size_t workspace_bytes, const sia_decode_options* opts,
                                     void* stream);

/* New composition for BASELINE configs 3 and 5 (paged pool + int8 + GQA group
 * per KV head); argument meaning follows paged_attention_flash_decode
 * (kernels/paged_flash_decode_kernel.py:107) and gqa_int8_flash_decode
 * (kernels/paged_flash_decode_int8_gqa_kernel.py:100).
 * k_pool,v_pool (num_pages,Hkv,page_size,D) int8; k_scale_pool,v_scale_pool
 * (num_pages,Hkv,page_size) f32|f16; page sizes as for
 * sia_paged_attention_flash_decode. */
int sia_paged_gqa_int8_flash_decode(const sia_tensor* q, const sia_tensor* k_pool,
                                    const sia_tensor* v_pool, const sia_tensor* k_scale_pool,
                                    const sia_tensor* v_scale_pool,
                                    const sia_tensor* block_table, const sia_tensor* kv_len,
                                    int32_t page_size, float sm_scale, const sia_tensor* out,
                                    void* workspace, size_t workspace_bytes,
                                    const sia_decode_options* opts, void* stream);

/* sia_paged_gqa_int8_flash_decode without a workspace argument: no
 * counterpart in the reference.  It is for callers that cannot allocate
 * device memory (code under HIP-graph capture, serving loops and harnesses
 * that forbid hipMalloc).  The split-K partials go to a static device array
 * of SIA_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds until
 * the process ends; nothing is allocated, freed or cleared per call.  A
 * geometry whose partials for one work-group per CU do not fit that array
 * fails with SIA_ERR_WORKSPACE (no valid head_dim/GQA shape does at 64 MiB).
 * Every call on a GPU shares that GPU's array, so calls that overlap on one
 * GPU (concurrent streams, threads) race: serialise them.  The array is
 * part of the library's code object, so every GPU on which any kernel of the
 * library is loaded holds its 64 MiB, whether or not this entry point is
 * called.  Arguments, results and errors are otherwise those of
 * sia_paged_gqa_int8_flash_decode. */
#define SIA_NOALLOC_SCRATCH_BYTES (64u << 20)
int sia_paged_gqa_int8_flash_decode_noalloc(const sia_tensor* q, const sia_tensor* k_pool,
                                            const sia_tensor* v_pool, const sia_tensor* k_scale_pool,
                                            const sia_tensor* v_scale_pool,
                                            const sia_tensor* block_table, const sia_tensor* kv_len,
                                            int32_t page_size, float sm_scale, const sia_tensor* out,
                                            const sia_decode_options* opts, void* stream);

/* Replaces attention_flash_triton (kernels/attention_kernel.py:235-305).
 * q (B,Hq,Tq,D), k,v (B,Hkv,Tk,D): f16|bf16|f32 views (one dtype), head_dim contiguous,
 * 16-byte aligned rows; out (B,Hq,Tq,D) view in q's dtype -- a transposed
 * view of a (B,Tq,Hq,D) buffer gives the reference's out_token_major layout.
 * causal != 0 applies the bottom-right mask: row i sees keys <= (Tk-Tq)+i;
 * rows that see no key are written as zeros.  head_dim 16, 32, 64, 128 or 256
 * (the reference's assert set, kernels/attention_kernel.py:273).
 * K rows (and float16 V rows at head_dim 32-128, which are read in place)
 * must lie at least one row's bytes and less than 2^31/64 bytes apart
 * (else SIA_ERR_UNSUPPORTED).
 * workspace: device memory of at least sia_prefill_workspace_size bytes
 * (256-byte aligned); it holds V converted to f16 in the kernel's block
 * layout (float16 V at head_dim 32-128 needs none: NULL, 0 is accepted
 * there) and is free again when the stream passes the call.  f32 inputs run in fp32 on the vector
 * ALUs and need no workspace (NULL, 0 is accepted). */
int sia_attention_flash_fwd(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, int32_t causal,
                            float sm_scale, const sia_tensor* out, void* workspace, size_t workspace_bytes,
                            void* stream);

/* sia_attention_flash_fwd with the rotary embedding of q applied as q is
 * loaded: replaces rope_triton (kernels/rope_kernel.py:261-285) on q followed
 * by attention_flash_triton (kernels/attention_kernel.py:235-305), the pair
 * the reference's prefill runs (ops/attention.py:291-292 then 327-330), in
 * one launch with no rotated copy of q.  k must already hold
 * rotated keys (sia_rope_kv_write with q NULL writes them to the cache).
 * Query row i of sequence b sits at position p = start_pos_host +
 * start_pos[b] + i, start_pos an int32 device tensor ((1,)/() shared or (B,)
 * per sequence, read on the device) or NULL (p = start_pos_host + i, checked
 * against the table rows on the host: SIA_ERR_INVALID_ARGUMENT).  cos, sin
 * as for sia_rope_qk (row p of the table, first D/2 columns, 16-byte aligned
 * rows) but in q's dtype or float32 (another dtype: SIA_ERR_UNSUPPORTED);
 * interleaved 0: pairs (i, i + D/2), 1: pairs (2i, 2i + 1).  The
 * rotation is sia_rope_qk's arithmetic and rounding, so the result equals
 * sia_rope_qk followed by sia_attention_flash_fwd bit for bit.  A device
 * position outside the table rotates q to zeros.  float16/bfloat16 only
 * (float32 q: SIA_ERR_UNSUPPORTED); workspace as for sia_attention_flash_fwd. */
int sia_attention_flash_fwd_rope(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, const sia_tensor* cos,
                                 const sia_tensor* sin, int32_t interleaved, const sia_tensor* start_pos,
                                 int32_t start_pos_host, int32_t causal, float sm_scale, const sia_tensor* out,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes sia_attention_flash_fwd needs for v of shape
 * (batch, kv_heads, kv_len, head_dim).  No reference counterpart: the
 * reference's Triton launch allocates nothing (kernels/attention_kernel.py:296). */
int sia_prefill_workspace_size(int64_t batch, int64_t kv_heads, int64_t kv_len, int64_t head_dim, size_t* bytes);

/* ------------------------------------------------------------ KV write path */

/* Replaces quantize_kv_int8 (model/kv_cache.py:58-67): per-vector symmetric
 * int8 over head_dim.  amax = max |x| clamped from below by 1e-8 (rounded to
 * x's dtype), scale = amax / 127 (fp32, correctly rounded), xi = round half
 * to even of x / scale, clamped to [-127, 127].
 * x (..., D) f16|bf16|f32 with 1..4 dims, head_dim contiguous and 16-byte
 * aligned rows; out_int8 same shape int8; out_scale x.shape[:-1] f16 (the
 * reference's KVCache dtype) or f32 (the paged pools' dtype). */
int sia_quantize_kv_int8(const sia_tensor* x, const sia_tensor* out_int8, const sia_tensor* out_scale, void* stream);

/* Writes new K/V tokens into a cache.  Replaces the write half of
 * KVCache.update (model/kv_cache.py:133-184), the decode-step
 * quantize_kv_int8 + index_copy_ scatter (ops/attention.py:217-228),
 * PagedKVCache.write_prefill (model/paged_kv_cache.py:89-109) and the
 * per-step paged write slot_for that the reference documents but does not
 * implement (model/paged_kv_cache.py:29-30).
 * k, v (B, H, T, D) f16|bf16|f32 (v may be NULL to write k alone).
 * Token t of (b, h) goes to position p = start_pos_host + start_pos[b] + t,
 * with start_pos an int32 device tensor ((1,)/() shared or (B,) per
 * sequence, read on the device: graph safe) or NULL (then p = start_pos_host
 * + t, checked against the cache length on the host).
 *  - block_table NULL: k_dst/v_dst are a contiguous cache (B' >= B, H, S, D)
 *    (a view into (L, B, H, S, D)); p must be < S.
 *  - block_table (B, max_blocks) int32: k_dst/v_dst are a paged pool
 *    (num_pages, H, page_size, D); p goes to page block_table[b][p / page_size]
 *    at offset p % page_size.
 * Destination dtype f16|bf16|f32 (value cast) or int8 (quantised exactly as
 * sia_quantize_kv_int8, with the per-token-per-head scale written to
 * k_scale_dst / v_scale_dst, shaped like the destination without head_dim,
 * f16 or f32).  Positions outside the destination (p >= capacity, page id
 * outside the pool) are skipped on the device, never written. */
int sia_kv_write(const sia_tensor* k, const sia_tensor* v, const sia_tensor* k_dst, const sia_tensor* v_dst,
                 const sia_tensor* k_scale_dst, const sia_tensor* v_scale_dst, const sia_tensor* block_table,
                 const sia_tensor* start_pos, int32_t start_pos_host, int32_t page_size, void* stream);

/* RoPE-K fused into the KV write, with q rotated in the same launch.
 * Replaces the captured decode step's apply_rope + quantize_kv_int8 + four
 * index_copy_ (ops/attention.py:200-228: rope at 202, writes at 217-228) and
 * the eager path's apply_rope + KVCache.update (ops/attention.py:290-300);
 * it is the fused RoPE-K write that model/paged_kv_cache.py:29-30 describes.
 * q (B, T, Hq, D) or NULL, k and v (B, T, Hkv, D) token-major, as the qkv
 * projection leaves them (strided slices are read in place); 16-byte aligned
 * rows.  Token t of sequence b has position p = start_pos_host + start_pos[b]
 * + t (start_pos as in sia_kv_write) and is rotated by table row p of
 * cos/sin ((Tc, D) or (Tc, D/2), f16|bf16|f32, 16-byte aligned with row
 * strides a multiple of 16 bytes, first D/2 columns read): pairs as in
 * sia_rope_qk (interleaved 0 or 1), the same fp32 arithmetic.  The rotated K
 * is rounded to k's dtype, then written like sia_kv_write writes k (cast, or
 * int8 with a per-token-per-head scale); v is written unrotated; q_out
 * (B, T, Hq, D), any strides with unit head_dim, receives the rotated q in
 * q's dtype.  Without start_pos (positions known on the host) every
 * position must have a table row, else SIA_ERR_INVALID_ARGUMENT.  With
 * start_pos (positions read on the device, where no error can be returned),
 * K/V rows whose position is outside the destination or the table are
 * skipped and q rows whose position is outside the table are written as
 * zeros: size the tables to the cache length. */
int sia_rope_kv_write(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, const sia_tensor* cos,
                      const sia_tensor* sin, int32_t interleaved, const sia_tensor* q_out, const sia_tensor* k_dst,
                      const sia_tensor* v_dst, const sia_tensor* k_scale_dst, const sia_tensor* v_scale_dst,
                      const sia_tensor* block_table, const sia_tensor* start_pos, int32_t start_pos_host,
                      int32_t page_size, void* stream);

/* Rotary position embedding of Q and K in one launch.  Replaces the Triton
 * kernel _rope_qk_fwd and its wrapper (kernels/rope_kernel.py:86-165,
 * 193-285), which ops/rope.py:206-226 (apply_rope) dispatches to.
 * q (B, T, Hq, D), k (B, T, Hkv, D), f16|bf16|f32, same dtype, D even; each
 * is read as B*T rows through one row stride (head_dim unit-stride, heads D
 * apart, stride(0) == T*stride(1) unless T == 1), so the Q/K slices of a
 * fused qkv buffer need no copy.  cos, sin (Tc, D) duplicated or (Tc, D/2)
 * raw, f16|bf16|f32, unit-stride rows; only the first D/2 columns are read;
 * row r of q/k uses position r % Tc.  interleaved 0: pairs (i, i + D/2)
 * (Llama/NeoX), 1: pairs (2i, 2i + 1) (GPT-J).  q_out, k_out contiguous,
 * the inputs' shape and dtype.  out_a = x_a cos - x_b sin and
 * out_b = x_b cos + x_a sin in fp32 with each product rounded (no fused
 * multiply-add), then rounded to the output dtype (nearest even). */
int sia_rope_qk(const sia_tensor* q, const sia_tensor* k, const sia_tensor* cos, const sia_tensor* sin,
                int32_t interleaved, const sia_tensor* q_out, const sia_tensor* k_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SIA_ATTENTION_H */
