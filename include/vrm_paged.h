/*
 * vrm_paged.h — C ABI of libvrm_paged.so, the gfx950 (MI355X) implementation of
 * VRAMancer's paged-attention decode over a quantized KV cache.
 *
 * Every entry point takes raw device pointers, explicit sizes and a HIP stream,
 * never allocates or frees device memory, and returns an int status:
 *      0              success (the kernels are enqueued on `stream`)
 *      < 0            invalid argument, detected on the host before any launch
 *      > 0            a hipError_t reported by the launch
 * vrm_last_error() returns a thread-local description of the last failure.
 * The library keeps no per-call state, so calls are reentrant; calls on one
 * stream are ordered by that stream.
 *
 * Pool layout (the reference's, core/paged_attention.py:321-330):
 *      kv_pool[P][L][2][KH][PS][D]    (index 2 selects K=0 / V=1)
 * with PS tokens per page (16 by default).  A sequence's logical page i lives in physical
 * page page_table[b][i]; tokens t < context_lens[b] are attended.
 * Float pools (f32, f16, bf16) keep each [PS][D] slice token-major, exactly as
 * the reference writes it.  The int8 and fp8 pools (this library's codecs,
 * written only by vrm_kv_quant_*) keep K token-major and store the V slice
 * tiled: the code of token t, dim d sits at byte
 *      ((t / 4 * 16 + d % 16) * (D / 16) + d / 16) * 4 + t % 4
 * of the slice, so that one decode lane loads its matrix-core operand for a
 * page as D / 4 consecutive bytes.
 */
#ifndef VRM_PAGED_H
#define VRM_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VRM_ABI_VERSION 2

/* Status codes (negative: rejected on the host, nothing was launched). */
#define VRM_OK 0
#define VRM_ERR_ARG (-1)          /* bad size, pointer, dtype or layer index */
#define VRM_ERR_UNSUPPORTED (-2)  /* valid request outside the compiled shapes */
#define VRM_ERR_WORKSPACE (-3)    /* workspace smaller than required */

/* Element type of the KV pool. */
typedef enum vrm_kv_dtype {
  VRM_KV_F32 = 0,      /* float32 pool                                        */
  VRM_KV_F16 = 1,      /* float16 pool                                        */
  VRM_KV_BF16 = 2,     /* bfloat16 pool                                       */
  VRM_KV_I8 = 3,       /* int8 codes, float32 scale per (page,layer,kv,head,token) */
  VRM_KV_FP8E4M3 = 4,  /* OCP e4m3fn codes, float32 scale per (page,layer,kv,head) */
  VRM_KV_I8_INLINE = 5,      /* VRM_KV_I8 codes and scales in the inline slab layout */
  VRM_KV_FP8E4M3_INLINE = 6  /* VRM_KV_FP8E4M3 codes and scales in the inline slab layout */
} vrm_kv_dtype;

/*
 * Inline slab layout of the int8 / fp8 pools (VRM_KV_*_INLINE).  The codes
 * and scales of one (page, layer) share one slab of vrm_kv_slab_bytes()
 * bytes, and the slabs lie layer by layer: slab (p, l) is at (l P + p) slab,
 * so that the P slabs of one layer form one contiguous run.  A slab holds for
 * each kv-head h in turn a record of
 *      K codes [PS][D] | V codes [PS][D] (tiled as above)
 *      | int8: K scales [PS], V scales [PS] float32 (PS (2 D + 8) bytes)
 *      | fp8:  K scale, V scale float32, zero bytes up to 2 PS D + 128
 * Code (p, l, kv, h, t, d) of the logical kv_pool[P][L][2][KH][PS][D] is at
 * byte (l P + p) slab + h record + kv PS D + (its place in the slice), and
 * the logical kv_scales[P][L][2][KH]([PS]) are float32s at the same slab and
 * record offsets plus kv PS (+ t) (int8) or kv (fp8) from
 * kv_scales = (char *)kv_pool + 2 PS D.  Every entry that takes a pool takes
 * these dtypes with kv_scales at exactly that address (anything else is
 * VRM_ERR_ARG).  No counterpart in the reference (whose pools are float
 * only, one page's layers side by side): a page of one layer is one run per
 * kv-head, and a layer's pages one run, which the balanced decodes sweep in
 * ascending page order (int8 14B shape, 48 layers, shuffled page table:
 * 98.0 -> 93.7 us per layer-step against the page-major float layout's
 * order).  The int8 pools of the Python layer use it by default; the fp8
 * pools do not (their few page scales read faster as a separate array in
 * the ragged work-item decode).
 */

/* Bytes of one (page, layer) slab of a pool of kv_dtype: 2 KH PS D times the
 * element size for the plain layouts (codes only: their scales live in
 * kv_scales), codes and scales for the inline layouts; 0 for a bad
 * argument. */
size_t vrm_kv_slab_bytes(int kv_dtype, int KH, int PS, int D);

/* Element type of new K/V rows handed to the quantizers. */
typedef enum vrm_src_dtype {
  VRM_SRC_F32 = 0,
  VRM_SRC_F16 = 1,
  VRM_SRC_BF16 = 2
} vrm_src_dtype;

typedef struct ihipStream_t* vrm_stream_t; /* == hipStream_t */

/* ABI version of the loaded library (== VRM_ABI_VERSION it was built with). */
int vrm_abi_version(void);

/* Thread-local text of the last error ("" when none). */
const char* vrm_last_error(void);

/* --------------------------------------------------------------------------
 * Paged decode attention.
 * -------------------------------------------------------------------------- */

/* Workspace sizing.  The decode cuts every sequence's pages into partitions
 * whose size the device derives from the context lengths; a batch never has
 * more than B + 2 * ceil(4096 / KH) partitions (work items).
 * vrm_paged_decode_num_splits returns that capacity per sequence,
 * ceil(capacity / B), and vrm_paged_decode_workspace_bytes the bytes for
 * B * nsplit items: a 256-byte aligned header of 16 + 2B + 1 ints (partition
 * geometry, written by the partition pass for the merge), then
 * [items][H][D] float32 accumulators and [items][H][2] (max, sum).  Both
 * depend only on the arguments (no device state); max_pp is the page-table
 * width. */
int vrm_paged_decode_num_splits(int B, int H, int KH, int max_pp, int page_size);
size_t vrm_paged_decode_workspace_bytes(int B, int H, int D, int nsplit);

/*
 * out[b][h][:] = softmax(scale * q[b][h] . K[b,kvh]^T) V[b,kvh] for one decode
 * token per sequence, kvh = h / (H / KH), reading K/V straight from the pages.
 *
 * Replaces the pybind entry `paged_attention_decode(query, kv_pool, page_table,
 * context_lens, layer_idx, scale)` of csrc/paged_attention_kernel.cu:445-499,
 * called from core/paged_attention_cuda.py:170-177; the int8 and fp8 pools
 * (kv_scales != NULL) have no counterpart in the reference and follow the
 * same signature with one extra scale pointer.
 *
 *   query        [B][H][D] float32
 *   kv_pool      [P][L][2][KH][PS][D] of kv_dtype
 *   kv_scales    VRM_KV_I8:      [P][L][2][KH][PS] float32 (per token)
 *                VRM_KV_FP8E4M3: [P][L][2][KH]     float32 (per page)
 *                float pools:    NULL
 *   page_table   [B][max_pp] int32; entries < 0 or >= P mark absent pages,
 *                whose tokens are skipped
 *   context_lens [B] int32; ctx <= 0 gives an all-zero output row
 *   out          [B][H][D] float32
 *   workspace    >= vrm_paged_decode_workspace_bytes(B, H, D, nsplit) bytes,
 *                nsplit = vrm_paged_decode_num_splits(...); may be NULL when
 *                that size is 0
 * Supported: any D <= 256 and any page size PS >= 1 (the reference's range,
 * csrc/paged_attention_kernel.cu:460-466), H % KH == 0; int8 / fp8 pools
 * need D % 16 == 0 and PS % 4 == 0 (their tiled V), and other shapes return
 * VRM_ERR_UNSUPPORTED.  Page 16 with D 64 / 128 / 256 runs the tuned
 * matrix-core kernels; every other shape a generic kernel.  int8 / fp8 pools
 * at D 64 .. 128 (multiples of 16) and page 16 hand page pairs to wavefronts
 * dynamically, so the last bits of an output may differ between calls.
 */
int vrm_paged_decode(const float* query, const void* kv_pool, const float* kv_scales,
                     const int32_t* page_table, const int32_t* context_lens,
                     float* out, void* workspace, size_t workspace_bytes,
                     int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                     int layer_idx, float scale, int kv_dtype, vrm_stream_t stream);

/*
 * vrm_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  No counterpart in the reference; it
 * allocates nothing and calls no allocating routine.  The split-K partials
 * live in a fixed array of VRM_NOALLOC_SCRATCH_BYTES inside the library, one
 * per GPU, held until the process ends; shapes whose workspace
 * (vrm_paged_decode_workspace_bytes with vrm_paged_decode_num_splits) is
 * larger are rejected with VRM_ERR_WORKSPACE.  All calls on one GPU share
 * that array: calls that overlap on one GPU (concurrent streams or threads)
 * race and must be serialised by the caller.  Same arguments, results and
 * supported shapes as vrm_paged_decode otherwise.
 */
/* The array is part of the code object that also holds the work-item and
 * TurboQuant decode kernels: any process that runs one of them on a GPU
 * holds these 64 MiB there until it ends, whether or not it calls this
 * entry. */
#define VRM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int vrm_paged_decode_noalloc(const float* query, const void* kv_pool, const float* kv_scales,
                             const int32_t* page_table, const int32_t* context_lens, float* out,
                             int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                             int layer_idx, float scale, int kv_dtype, vrm_stream_t stream);

/*
 * vrm_paged_decode for batches whose sequences have about equal context
 * lengths (the caller knows them on the host; the page manager does).  One
 * workgroup per (sequence, kv-head or head chunk) splits the sequence's pages
 * over its wavefronts and merges their partials in LDS, writing out directly:
 * no workspace, no separate merge pass.  A workgroup reads its sequence's
 * whole pages in ascending page id (sorted in LDS), so that over the inline
 * layout's layer-major slabs the workgroups sweep a layer's pages together.
 * Correct for any lengths; its time
 * follows the longest sequence, so ragged batches belong on vrm_paged_decode,
 * which balances work items across sequences.  lse (nullable) receives
 * ln sum_t exp(scale q.k_t) per (b, h) as in vrm_paged_decode_lse.  No
 * counterpart in the reference (whose kernel is one warp per (head, sequence),
 * csrc/paged_attention_kernel.cu:445-499, with no split).
 * Supported: int8 and fp8 pools, D in {64, 80, 96, 112, 128}, PS == 16, and page tables
 * narrow enough for a workgroup's LDS copy of one row (max_pp up to ~12000 at
 * D = 128); other requests return VRM_ERR_UNSUPPORTED.
 */
int vrm_paged_decode_balanced(const float* query, const void* kv_pool, const float* kv_scales,
                              const int32_t* page_table, const int32_t* context_lens, float* out, float* lse,
                              int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                              int layer_idx, float scale, int kv_dtype, vrm_stream_t stream);

/*
 * Measurement aid, no counterpart in the reference: the balanced decode's
 * own loads (same grid, addresses, order, register ring and page hand-out)
 * with the computation left out; a checksum of the loaded words lands in
 * out (values meaningless).  Its time is what the decode's access pattern
 * alone costs on this GPU, the ceiling against which the decode's own time
 * is judged.  Same arguments and support as vrm_paged_decode_balanced.
 */
int vrm_paged_decode_balanced_loads(const float* query, const void* kv_pool, const float* kv_scales,
                                    const int32_t* page_table, const int32_t* context_lens, float* out,
                                    int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                                    int layer_idx, float scale, int kv_dtype, vrm_stream_t stream);

/*
 * The two passes of vrm_paged_decode, for callers that schedule them
 * separately (and for timing the dominant pass on its own):
 * vrm_paged_decode_partitions writes per-partition (max, sum, unnormalised
 * accumulator) into the workspace; vrm_paged_decode_merge combines them into
 * out.  Same arguments and workspace contract as vrm_paged_decode; merge only
 * reads query/kv_pool/kv_scales for argument checks, never their contents.
 * No counterpart in the reference, whose kernel is single-pass.
 */
int vrm_paged_decode_partitions(const float* query, const void* kv_pool, const float* kv_scales,
                                const int32_t* page_table, const int32_t* context_lens,
                                void* workspace, size_t workspace_bytes,
                                int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                                int layer_idx, float scale, int kv_dtype, vrm_stream_t stream);
int vrm_paged_decode_merge(const int32_t* context_lens, float* out,
                           const void* workspace, size_t workspace_bytes,
                           int B, int H, int KH, int D, int PS, int max_pp, vrm_stream_t stream);

/*
 * vrm_paged_decode that also writes lse[b][h] = ln sum_t exp(scale q.k_t)
 * over the attended tokens (-inf when none), so that attentions over
 * disjoint token sets can be merged (vrm_attn_combine).  No counterpart in
 * the reference; used by the Hugging Face cache integration to merge the
 * compressed pages with the uncompressed recent tokens
 * (core/turboquant_cache.py:176-196 concatenates them instead).
 */
int vrm_paged_decode_lse(const float* query, const void* kv_pool, const float* kv_scales,
                         const int32_t* page_table, const int32_t* context_lens, float* out,
                         float* lse, void* workspace, size_t workspace_bytes, int B, int H, int KH,
                         int D, int PS, int L, int P, int max_pp, int layer_idx, float scale,
                         int kv_dtype, vrm_stream_t stream);

/*
 * out = (e^(lse1 - m) out1 + e^(lse2 - m) out2) / (e^(lse1 - m) + e^(lse2 - m)),
 * m = max(lse1, lse2), row by row ([rows][D] float32 outputs, [rows] lse):
 * the attention over the union of two disjoint token sets from the
 * attentions over each.  A row with both lse = -inf gives zeros; lse_out
 * (optional) gets the union's lse.  No counterpart in the reference.
 */
int vrm_attn_combine(const float* out1, const float* lse1, const float* out2, const float* lse2,
                     long long rows, int D, float* out, float* lse_out, vrm_stream_t stream);

/*
 * Same attention over the reference's asymmetric 4-bit pool:
 *   value(d) = (nibble(d) - zero[g]) * scale[g],  g = d / 32,
 *   byte j of a row holds d = 2j in its low nibble and d = 2j+1 in its high one.
 * Replaces the pybind entry `paged_attention_decode_q4` of
 * csrc/paged_attention_kernel.cu:502-549 (wrapper core/paged_attention_cuda.py:238-288).
 *   kv_pool_q4  [P][L][2][KH][PS][D/2] uint8
 *   kv_scales, kv_zeros [P][L][2][KH][PS][D/32] float16 (passed as uint16 bits)
 * Supported: D % 32 == 0 (D <= 256), any page size.
 */
int vrm_paged_decode_q4(const float* query, const uint8_t* kv_pool_q4,
                        const uint16_t* kv_scales, const uint16_t* kv_zeros,
                        const int32_t* page_table, const int32_t* context_lens,
                        float* out, void* workspace, size_t workspace_bytes,
                        int B, int H, int KH, int D, int PS, int L, int P, int max_pp,
                        int layer_idx, float scale, vrm_stream_t stream);

/* --------------------------------------------------------------------------
 * Quantize-on-append into int8 / fp8 pools.  No counterpart exists in the
 * reference (core/kv_quantizer.py is TurboQuant-only); the write itself
 * replaces the raw index-put of PagedKVCacheManager.write_kv
 * (core/paged_attention.py:611-612: pool[page, layer, 0|1, :, slot, :] = k|v).
 * -------------------------------------------------------------------------- */

/*
 * Writes N new tokens.  Token n goes to (page_ids[n], slots[n]) of layer
 * layer_idx; key/value are [N][KH][D] of src_dtype.
 *   VRM_KV_I8:      per (token, head) amax over D; scale = amax / 127;
 *                   code = clamp(round_half_even(x / scale), -127, 127);
 *                   amax == 0 gives scale 0 and codes 0.
 *   VRM_KV_FP8E4M3: the page's per-head scale only grows.  With old scale s
 *                   (taken as 0 when slots[n] == 0) and a = amax(x) / 448:
 *                   s' = max(s, a); codes already in slots < slots[n] are
 *                   re-encoded as e4m3(fp32(e4m3 code) * s / s') when s' > s,
 *                   then the new row is e4m3(x / s') (round to nearest even).
 *                   Several tokens of one call must not share a page.
 * kv_pool/kv_scales as in vrm_paged_decode.  Supported: D a multiple of 16 up
 * to 256, PS a multiple of 4.
 */
int vrm_kv_quant_append(const void* key, const void* value, int src_dtype,
                        const int32_t* page_ids, const int32_t* slots, int N,
                        void* kv_pool, float* kv_scales, int kv_dtype,
                        int KH, int D, int PS, int L, int P, int layer_idx,
                        vrm_stream_t stream);

/*
 * Bulk (prefill) write of whole pages.  key/value are [NP][KH][PS][D] of
 * src_dtype; page n goes to physical page page_ids[n] and holds n_valid[n]
 * tokens (slots >= n_valid are written as code 0).
 *   VRM_KV_I8:      as vrm_kv_quant_append, per token.
 *   VRM_KV_FP8E4M3: scale = amax over the valid tokens of the page-head / 448.
 */
int vrm_kv_quant_pages(const void* key, const void* value, int src_dtype,
                       const int32_t* page_ids, const int32_t* n_valid, int NP,
                       void* kv_pool, float* kv_scales, int kv_dtype,
                       int KH, int D, int PS, int L, int P, int layer_idx,
                       vrm_stream_t stream);

/*
 * Dequantizes pages of a quantized pool to float32: for each n,
 * out[n][2][KH][PS][D] = codes of (page_ids[n], layer_idx) * scale.
 * Debug/offload helper; decode never materializes this.
 */
int vrm_kv_dequant_pages(const void* kv_pool, const float* kv_scales, int kv_dtype,
                         const int32_t* page_ids, int NP, float* out,
                         int KH, int D, int PS, int L, int P, int layer_idx,
                         vrm_stream_t stream);

/* --------------------------------------------------------------------------
 * TurboQuant (randomized Hadamard + PolarQuant + QJL) codec.
 * -------------------------------------------------------------------------- */

/*
 * Compresses N rows of head_dim values, following the CPU path of
 * KVCacheCompressor.compress (core/kv_quantizer.py:391-417): pad to
 * padded_dim, rotate, 7-level polar encode, bin angles, decode with the fp32
 * radius, QJL-sign the residual.  Replaces the pybind entry `compress` of
 * csrc/turboquant_kernel.cu:410-450 (wrapper core/turboquant_cuda.py:124-174).
 *   kv          [N][head_dim] of src_dtype
 *   signs       [padded_dim] float32 (+-1), jl [qjl_dim][padded_dim] float32
 *   angle_lut   [2][2][2^bits] float32: {cos, sin} of the bin centres of
 *               level 0 and of levels >= 1, as the host computes them
 *   radius      [N] float16 bits; angles [N][padded_dim-1] uint8, level-major
 *               (level 0 first); qjl_signs [N][qjl_dim] uint8 (0/1);
 *               qjl_norms [N] float16 bits
 * Supported: padded_dim a power of two from 2 to 256 (head_dim 1 .. 256, as
 * the reference pads any head_dim to 2^ceil(log2 max(head_dim, 2)),
 * core/kv_quantizer.py:225), 1 <= bits <= 8, qjl_dim <= 4 padded_dim.
 */
int vrm_turboquant_compress(const void* kv, int src_dtype, int N, int head_dim,
                            int padded_dim, int n_levels, int bits, int qjl_dim,
                            const float* signs, const float* jl, const float* angle_lut,
                            uint16_t* radius, uint8_t* angles, uint8_t* qjl_signs,
                            uint16_t* qjl_norms, vrm_stream_t stream);

/*
 * out[N][head_dim] float32 = unrotate(polar_decode(radius, angles)), no QJL
 * (core/kv_quantizer.py:481-500).  Replaces the pybind entry `decompress` of
 * csrc/turboquant_kernel.cu:453-481.  With rotated != 0 the inverse rotation
 * is skipped and out is [N][padded_dim] = polar_decode(radius, angles), the
 * key reconstruction that KVCacheCompressor.attention_score dots with the
 * rotated query (core/kv_quantizer.py:523-527).
 */
int vrm_turboquant_decompress(const uint16_t* radius, const uint8_t* angles, int N,
                              int head_dim, int padded_dim, int n_levels, int bits,
                              const float* signs, const float* angle_lut, float* out,
                              int rotated, vrm_stream_t stream);

/*
 * scores[M][N] float32 = out_scale * (q_rot . k_polar + QJL correction) for M
 * query rows q [M][head_dim] float32 against N compressed keys in the raw
 * format of vrm_turboquant_compress: KVCacheCompressor.attention_score
 * (core/kv_quantizer.py:502-535; q_rot = rotate(pad(q)), k_polar the polar
 * decode from the fp16 radius, correction = (q_rot JL^T . (2 s - 1)) *
 * sqrt(pi / 2) / qjl_dim * norm).  Replaces the tensor-op path of
 * CUDATurboQuantOps.attention_score_gpu (core/turboquant_cuda.py:208-255),
 * with the rotated query in both terms as the reference's CPU path has it.
 * workspace: >= vrm_turboquant_score_workspace_bytes(M, padded_dim, qjl_dim)
 * bytes (the rotated and projected queries).  M <= 65535.
 */
size_t vrm_turboquant_score_workspace_bytes(int M, int padded_dim, int qjl_dim);
int vrm_turboquant_score(const float* q, int M, const uint16_t* radius, const uint8_t* angles,
                         const uint8_t* qjl_signs, const uint16_t* qjl_norms, int N, int head_dim,
                         int padded_dim, int n_levels, int bits, int qjl_dim, const float* signs,
                         const float* jl, const float* angle_lut, float out_scale, float* workspace,
                         size_t workspace_bytes, float* scores, vrm_stream_t stream);

/*
 * Top-k ("sparse V") attention over explicit scores: for each row m of
 * scores[M][N] (row stride ld_scores), the k largest scores S_m are kept and
 *   out[m][:] = sum_{n in S_m} e^(s_mn - max) values[n][:] / sum_{n in S_m} e^(s_mn - max),
 * the renormalised top-k softmax weights of KVCacheCompressor.sparse_v_attend
 * (core/kv_quantizer.py:537-562) and of compute_attention_turbo with
 * sparse_v_ratio < 1 (core/paged_attention.py:1384-1400).  Of scores equal to
 * the k-th largest, the lowest-indexed are kept.  k = N is the dense
 * softmax(scores) values.  values [N][D] (row stride ld_values), out [M][D]
 * (row stride ld_out), float32; 1 <= k <= N.
 * workspace: >= vrm_topk_attend_workspace_bytes(M, k) bytes (selection,
 * kept indices and weights, and the partial sums of the weighted sum).
 */
size_t vrm_topk_attend_workspace_bytes(int M, int k);
int vrm_topk_attend(const float* scores, int M, int N, long long ld_scores, int k, const float* values,
                    int D, long long ld_values, float* out, long long ld_out, void* workspace,
                    size_t workspace_bytes, vrm_stream_t stream);

/*
 * Packed code format of KVCacheCompressor (core/kv_quantizer.py:46-105,
 * 337-371): each of `rows` rows of M uint8 values contributes the low `bits`
 * bits of every value, most significant bit first; the row's bit stream fills
 * ceil(M * bits / 8) bytes from bit 7 of byte 0, the last byte zero-padded.
 * QJL signs use bits = 1, angle bins bits = bits_per_angle over a row's
 * level-major bins.  vrm_unpack_bits is the inverse.  1 <= bits <= 8.
 */
int vrm_pack_bits(const uint8_t* vals, long long rows, int M, int bits, uint8_t* packed,
                  vrm_stream_t stream);
int vrm_unpack_bits(const uint8_t* packed, long long rows, int M, int bits, uint8_t* vals,
                    vrm_stream_t stream);

/* --------------------------------------------------------------------------
 * TurboQuant pages.  The reference keeps TurboQuant-compressed K/V in Python
 * dicts per (page, layer, slot) (core/paged_attention.py:568-675, 1420-1496)
 * and attends them with compute_attention_turbo (:1259-1418).  Here the same
 * codes live in a device pool tq_pool[P][L][2][KH][slice] (bytes), one slice
 * of vrm_tq_slice_bytes_ps() per (page, layer, K/V, kv-head) holding the
 * page's tokens: angle bins, fp16 radius and, for K, the QJL sign bits and the
 * fp16 residual norm.  Every compressor setting of the reference's
 * KVCacheCompressor (core/kv_quantizer.py:205-240) with head_dim 1..256
 * (padded_dim 2, 4, ..., 256), 1..8 bits per angle and qjl_dim 1..256 is
 * served, at any page size.  head_dim 33..128 with the compressor's default
 * qjl_dim (padded_dim / 2: 32 or 64), 2..4 bits and 16-token pages use tuned
 * slices (angle bins in a lane-friendly order of the reference's
 * padded_dim - 1 bins) and decode kernel; every other setting a generic
 * slice of per-token records (level-major angle bits, sign bits, radius,
 * norm).  signs / jl / angle_lut are the compressor's buffers and the
 * {cos, sin} table of vrm_turboquant_compress.
 * -------------------------------------------------------------------------- */

/* Bytes of one (page, layer, K/V, kv-head) slice of page_size tokens; 0 for
 * an unsupported setting.  No reference counterpart: the reference keeps
 * per-slot dicts (core/paged_attention.py:568-675), the pool needs a size. */
size_t vrm_tq_slice_bytes_ps(int head_dim, int bits, int qjl_dim, int page_size);

/* vrm_tq_slice_bytes_ps at the default 16-token page. */
size_t vrm_tq_slice_bytes(int head_dim, int bits, int qjl_dim);

/*
 * Compresses N new tokens (key/value [N][KH][D] of src_dtype) into slot
 * slots[n] of page page_ids[n], layer layer_idx.  Codes are those of
 * vrm_turboquant_compress (the reference's KVCacheCompressor.compress CPU
 * path); V rows store angles and radius only (the attention never reads a
 * value's QJL fields).  Replaces write_kv's enqueue + flush_compression
 * (core/paged_attention.py:615-675).  Rows aimed at pages outside [0, P) or
 * slots outside [0, PS) are dropped.
 */
int vrm_tq_quant_append(const void* key, const void* value, int src_dtype,
                        const int32_t* page_ids, const int32_t* slots, int N,
                        uint8_t* tq_pool, int KH, int D, int PS, int L, int P, int layer_idx,
                        int bits, int qjl_dim, const float* signs, const float* jl,
                        const float* angle_lut, vrm_stream_t stream);

/*
 * Bulk write of whole pages (key/value [NP][KH][PS][D]); page n holds
 * n_valid[n] tokens, later slots get zero codes.  Replaces compress_page_bulk
 * (core/paged_attention.py:1420-1496).
 */
int vrm_tq_quant_pages(const void* key, const void* value, int src_dtype,
                       const int32_t* page_ids, const int32_t* n_valid, int NP,
                       uint8_t* tq_pool, int KH, int D, int PS, int L, int P, int layer_idx,
                       int bits, int qjl_dim, const float* signs, const float* jl,
                       const float* angle_lut, vrm_stream_t stream);

/*
 * compress_page_bulk's device work (core/paged_attention.py:1420-1496): reads
 * pages page_ids[n] of layer layer_idx from a float pool kv_pool[P][L][2][KH]
 * [PS][D] (kv_dtype f32, f16 or bf16, the manager's raw pool) and writes
 * their codes into the same (page, layer) of tq_pool; page n holds n_valid[n]
 * tokens, later slots get zero codes.  Codes as vrm_tq_quant_pages.
 */
int vrm_tq_compress_pool(const void* kv_pool, int kv_dtype, const int32_t* page_ids,
                         const int32_t* n_valid, int NP, uint8_t* tq_pool, int KH, int D, int PS,
                         int L, int P, int layer_idx, int bits, int qjl_dim, const float* signs,
                         const float* jl, const float* angle_lut, vrm_stream_t stream);

/*
 * Reads pages back in the reference's raw code format: row
 * ((n * 2 + kv) * KH + h) * PS + t gets radius (fp16 bits), the
 * padded_dim - 1 level-major bins, qjl_dim sign bytes and the norm (V rows:
 * zero signs / norm).
 * Inspection and offload helper.
 */
int vrm_tq_read_pages(const uint8_t* tq_pool, const int32_t* page_ids, int NP,
                      int KH, int D, int PS, int L, int P, int layer_idx, int bits, int qjl_dim,
                      uint16_t* radius, uint8_t* angles, uint8_t* qjl_signs, uint16_t* qjl_norms,
                      vrm_stream_t stream);

/*
 * Paged decode over TurboQuant pages: for query head h (kv-head h / (H / KH)),
 * out = softmax(scale * score) V with score_t = q_rot . k_polar_t + the QJL
 * correction, and V the decompressed values, as
 * PagedKVCacheManager.compute_attention_turbo (core/paged_attention.py:
 * 1259-1418) with dense values (sparse_v_ratio 1.0).  Workspace and split
 * contract as vrm_paged_decode.
 */
int vrm_paged_decode_tq(const float* query, const uint8_t* tq_pool, const int32_t* page_table,
                        const int32_t* context_lens, float* out, void* workspace, size_t workspace_bytes,
                        int B, int H, int KH, int D, int PS, int L, int P, int max_pp, int layer_idx,
                        float scale, int bits, int qjl_dim, const float* signs, const float* jl,
                        const float* angle_lut, vrm_stream_t stream);

/* --------------------------------------------------------------------------
 * Paged cache manager support (PagedKVCacheManager, core/paged_attention.py).
 * -------------------------------------------------------------------------- */

/*
 * Block-table build of compute_attention_decode (core/paged_attention.py:
 * 1226-1248): request b's pages are flat_pages[offsets[b] .. offsets[b+1]),
 * offsets has B + 1 entries.  Writes page_table[b][p] = its p-th page for
 * p below the count and -1 up to max_pp, and context_lens[b] =
 * num_tokens[b].  A list that overruns the flat array or max_pp is cut
 * (entries past max_pp are not written; a malformed (offsets[b],
 * offsets[b+1]) pair gives a row of -1).
 */
int vrm_build_block_table(const int32_t* flat_pages, int n_flat, const int32_t* offsets,
                          const int32_t* num_tokens, int B, int max_pp, int32_t* page_table,
                          int32_t* context_lens, vrm_stream_t stream);

/*
 * Raw write of N tokens into a float pool: replaces write_kv's index-put
 * (core/paged_attention.py:611-612, pool[page, layer, 0|1, :, slot, :] =
 * key|value).  key/value are [N][KH][D] of src_dtype; kv_dtype is VRM_KV_F32,
 * VRM_KV_F16 or VRM_KV_BF16; conversions round to nearest even.  Rows aimed
 * at pages outside [0, P) or slots outside [0, PS) are dropped.
 */
int vrm_kv_write(const void* key, const void* value, int src_dtype, const int32_t* page_ids,
                 const int32_t* slots, int N, void* kv_pool, int kv_dtype, int KH, int D, int PS,
                 int L, int P, int layer_idx, vrm_stream_t stream);

/*
 * vrm_paged_decode_tq plus the lse output of vrm_paged_decode_lse.  With
 * with_qjl != 0 the scores are compute_attention_turbo's (QJL-corrected);
 * with with_qjl == 0 they are q . decompress(k), the keys the reference's
 * Hugging Face cache hands to the model's attention
 * (core/turboquant_cache.py:135-138, 176-186).
 */
int vrm_paged_decode_tq_lse(const float* query, const uint8_t* tq_pool, const int32_t* page_table,
                            const int32_t* context_lens, float* out, float* lse, void* workspace,
                            size_t workspace_bytes, int B, int H, int KH, int D, int PS, int L, int P,
                            int max_pp, int layer_idx, float scale, int bits, int qjl_dim,
                            const float* signs, const float* jl, const float* angle_lut,
                            int with_qjl, vrm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VRM_PAGED_H */
