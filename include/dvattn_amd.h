/*
 * dvattn_amd.h -- C ABI of the MI355X (gfx950) DVAttn library, libdvattn_amd.so.
 *
 * Drop-in replacement for the compute entry points behind the reference's
 * `libdvatt` torch operators.  Every function here is plain C: raw device
 * pointers, int sizes, a caller-owned device workspace and a HIP stream passed
 * as `void*`.  Nothing throws across this boundary; each call returns a
 * dvattn_status and, on failure, leaves a message for dvattn_last_error().
 *
 * Reference interfaces replaced (paths in the reference repository):
 *   dvattn_paged_sdpa        <- op `dvattn_paged_sdpa`, src/binding.cu:412-413,151-203
 *                               (+ rope_gpu src/rope.cuh:54-65 and
 *                               paged_v21::dvattn_paged_attention_gpu
 *                               src/kernels/paged_kernel_v21.cuh:377-431)
 *   dvattn_varlen_paged_sdpa <- op `dvattn_varlen_paged_sdpa`, src/binding.cu:418-420,249-296
 *                               (+ rope_varlen_gpu src/rope.cuh:102-114 and
 *                               src/kernels/varlen_paged_kernel_v21.cuh:373-428)
 *   dvattn_sdpa              <- op `dvattn_sdpa`, src/binding.cu:410-411,79-149
 *                               (+ v21::dvattn_attention_gpu src/kernels/kernel_v21.cuh:369-414)
 *   dvattn_fused             <- op `dvattn_fused`, src/binding.cu:415-416,356-372
 *   dvattn_rope              <- op `dvattn_rope`, src/binding.cu:414,41-77 (rope_gpu)
 *   dvattn_varlen_rope       <- op `dvattn_varlen_rope`, src/binding.cu:417,205-247
 *   dvattn_shape             <- struct Shape, src/common.h:5-20
 * and, around the path (the reference does these in Python):
 *   dvattn_paged_kv_append   <- python/dvattn/attention.py:304 + 141-152 (key rotation and
 *                               cache append of a decode step), 245-251 (merge_caches)
 *   dvattn_view_metadata     <- python/dvattn/attention.py:158-186 (per-view locations,
 *                               cos/sin)
 *
 * Semantics (identical to the reference operators):
 *   - GQA factor 16 (Hq == 16*Hkv) and head dims E == Ev == 128 only; other
 *     shapes are rejected with DVATTN_ERR_UNSUPPORTED (the reference printed a
 *     message and returned/no-op'd, paged_kernel_v21.cuh:426-429, kernel_v21.cuh:410-413).
 *   - Query rotation: dims e < R use x*cos - rotate_half(x)*sin with the first
 *     R/2 entries of each cos/sin row (full width [.., R] for paged/contiguous,
 *     half width [.., R/2] for varlen); dims >= R are copied.  fp32 math,
 *     rotated query rounded to the storage type before the dot products.
 *   - Key l of view f is visible to a query iff 0 <= l <= locations[f, row]
 *     and l < fragment_lengths[f]; one softmax over all visible keys of all
 *     views; fp32 accumulation; a query row with no visible key outputs zeros.
 *   - Paged views are laid out back to back in each sequence's logical token
 *     stream: view f starts at sum_{g<f} fragment_lengths[g]; logical position
 *     p lives in page block_tables[w, p / block_size], row p % block_size of a
 *     [num_blocks, block_size, Hkv, E] cache.
 *   - Keys whose logical page is beyond the block_tables row, or whose page id
 *     is outside [0, num_blocks), are treated as not visible (the reference
 *     reads out of bounds there).
 *
 * Alignment (checked; the reference's kernels assumed 16-byte vectors,
 * paged_kernel_v21.cuh:58-62, without checking): the attention entry points
 * (dvattn_paged_sdpa[_noalloc], dvattn_varlen_paged_sdpa, dvattn_sdpa,
 * dvattn_fused) need out, queries, rotated_queries, k_cache, v_cache, every
 * key/value fragment and the workspace 16-byte aligned and the int32 / fp32
 * arrays 4-byte aligned; dvattn_rope, dvattn_varlen_rope and
 * dvattn_paged_kv_append need each array aligned to its element size.  A
 * pointer off its alignment returns DVATTN_ERR_INVALID, naming the argument.
 * Tensors from a device allocator, and views of them that start on a row of
 * the last dimension, always qualify.
 */
#ifndef DVATTN_AMD_H
#define DVATTN_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DVATTN_ABI_VERSION 1

#if defined(__GNUC__) || defined(__clang__)
#define DVATTN_API __attribute__((visibility("default")))
#else
#define DVATTN_API
#endif

/* Storage type of queries / keys / values / outputs (cos/sin are always fp32,
 * index tensors int32), binding.cu:14-38. */
typedef enum dvattn_dtype {
    DVATTN_F32 = 0,
    DVATTN_F16 = 1,
    DVATTN_BF16 = 2
} dvattn_dtype;

typedef enum dvattn_status {
    DVATTN_OK = 0,
    DVATTN_ERR_INVALID = 1,     /* bad argument (null pointer, inconsistent sizes) */
    DVATTN_ERR_UNSUPPORTED = 2, /* shape/dtype outside what the kernels implement */
    DVATTN_ERR_WORKSPACE = 3,   /* workspace smaller than the *_workspace_size query */
    DVATTN_ERR_HIP = 4          /* a HIP runtime call failed */
} dvattn_status;

/* Launch descriptor, mirrors Shape (src/common.h:5-20).  Fields an entry point
 * does not use are ignored. */
typedef struct dvattn_shape {
    int F;                  /* views ("fragments") */
    int W;                  /* sequences ("workers") */
    int Hq;                 /* query heads (16 * Hkv) */
    int Hkv;                /* key/value heads */
    int E;                  /* q/k head dim (128) */
    int Ev;                 /* v head dim (128) */
    int S;                  /* query tokens per sequence (paged / contiguous) */
    int block_size;         /* page size in tokens (paged, varlen) */
    int max_blocks_per_seq; /* block_tables row length (paged, varlen) */
    int total_q_tokens;     /* T (varlen) */
    int num_blocks;         /* pages in k_cache / v_cache (paged, varlen) */
    int rotary_dim;         /* R (even, <= E; 0 = no rotation) */
} dvattn_shape;

/* Last error message of the calling thread ("" if none). */
DVATTN_API const char* dvattn_last_error(void);
DVATTN_API int dvattn_abi_version(void);

/* Process-wide switches.  No counterpart in the reference (its kernels have no
 * such choices).  Each starts from an environment variable, read once at first
 * use; dvattn_set_option replaces the value for all later calls (set it while
 * no other thread is inside a call, or those calls may see either value).
 *   "small_path"  (DVATTN_SMALL_PATH: 0/"0" off, 1 auto = default, 2/"require",
 *                  3/"force"): the single-launch path of dvattn_sdpa /
 *                  dvattn_fused; require fails a call it cannot take with
 *                  DVATTN_ERR_UNSUPPORTED, force takes it past its workgroup limit.
 * dvattn_get_option returns the current value, -1 for an unknown name. */
DVATTN_API dvattn_status dvattn_set_option(const char* name, int value);
DVATTN_API int dvattn_get_option(const char* name);

/* ---- paged decode attention with fused query RoPE --------------------------
 * out [W,Hq,S,Ev] T; locations [F,W,S] i32; queries [W,Hq,S,E] T;
 * cosines/sines [F,W,S,R] f32; fragment_lengths [F] i32 (device);
 * k_cache [num_blocks,block_size,Hkv,E] T; v_cache [num_blocks,block_size,Hkv,Ev] T;
 * block_tables [W,max_blocks_per_seq] i32.  All contiguous, on one device.
 * Replaces binding.cu:151-203 / paged_kernel_v21.cuh:377-431. */
DVATTN_API size_t dvattn_paged_sdpa_workspace_size(int dtype, const dvattn_shape* shape, int device);
DVATTN_API dvattn_status dvattn_paged_sdpa(int dtype, void* out, float scale, const int* locations,
                                const void* queries, const float* cosines, const float* sines,
                                const int* fragment_lengths, const void* k_cache, const void* v_cache,
                                const int* block_tables, const dvattn_shape* shape,
                                void* workspace, size_t workspace_bytes, void* stream);

/* ---- paged decode attention without allocation -----------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  Same arguments, checks and results as dvattn_paged_sdpa,
 * minus the workspace: the partial results and merge directory live in a static
 * device array of DVATTN_NOALLOC_SCRATCH_BYTES that each GPU the library runs on
 * holds until the process ends.  A shape whose dvattn_paged_sdpa_workspace_size
 * exceeds it is rejected with DVATTN_ERR_WORKSPACE.  The call allocates nothing
 * (no hipMalloc, no allocating library routine).  Every call on a GPU uses that
 * GPU's one array: calls that overlap on one GPU (two streams or threads at
 * once) race and must be serialised by the caller. */
#define DVATTN_NOALLOC_SCRATCH_BYTES (64u << 20)
DVATTN_API dvattn_status dvattn_paged_sdpa_noalloc(int dtype, void* out, float scale, const int* locations,
                                        const void* queries, const float* cosines, const float* sines,
                                        const int* fragment_lengths, const void* k_cache,
                                        const void* v_cache, const int* block_tables,
                                        const dvattn_shape* shape, void* stream);

/* ---- varlen paged decode attention with fused query RoPE -------------------
 * out [T,Hq,Ev] T; locations [F,T] i32 (a view with locations < 0 is skipped);
 * queries [T,Hq,E] T; cosines/sines [F,T,R/2] f32 (half width);
 * cu_seqlens_q [W+1] i32: token t belongs to the first sequence i with
 * t < cu_seqlens_q[i+1] (sequence 0 if none); cu_seqlens_k is accepted and,
 * as in the reference (binding.cu:279,290), not read.  16-bit calls with
 * T >= 2W (and W <= 4096) read each sequence's K/V once per group of up to 16
 * of its tokens (the workspace size follows the same rule); other calls once
 * per token, as the reference does.
 * Replaces binding.cu:249-296 / varlen_paged_kernel_v21.cuh:373-428. */
DVATTN_API size_t dvattn_varlen_paged_sdpa_workspace_size(int dtype, const dvattn_shape* shape, int device);
DVATTN_API dvattn_status dvattn_varlen_paged_sdpa(int dtype, void* out, float scale, const int* locations,
                                       const void* queries, const float* cosines, const float* sines,
                                       const int* fragment_lengths, const void* k_cache,
                                       const void* v_cache, const int* block_tables,
                                       const int* cu_seqlens_q, const int* cu_seqlens_k,
                                       const dvattn_shape* shape, void* workspace,
                                       size_t workspace_bytes, void* stream);

/* ---- contiguous-view attention on already-rotated queries ------------------
 * out [W,Hq,S,Ev] T; locations [F,W,S]; rotated_queries [F,W,Hq,S,E] T;
 * fragment_lengths [F] i32 (device).  key_fragments[f] / value_fragments[f]
 * (host arrays of F device pointers) point at [B_f,Hkv,L_f,E|Ev] T tensors;
 * fragment_tokens[f] = L_f and fragment_batch[f] = B_f (host arrays).  B_f is
 * W, or 1 for a fragment shared by every sequence (the PyTorch reference
 * broadcasts it, attention.py:45,53).  Visible keys are also bounded by L_f.
 * Replaces binding.cu:79-149 / kernel_v21.cuh:369-414. */
DVATTN_API size_t dvattn_sdpa_workspace_size(int dtype, const dvattn_shape* shape, int device);
DVATTN_API dvattn_status dvattn_sdpa(int dtype, void* out, float scale, const int* locations,
                          const void* rotated_queries, const int* fragment_lengths,
                          const void* const* key_fragments, const void* const* value_fragments,
                          const int* fragment_tokens, const int* fragment_batch,
                          const dvattn_shape* shape, void* workspace, size_t workspace_bytes,
                          void* stream);

/* ---- rope + contiguous attention (dvattn_fused) -----------------------------
 * Writes rotated_queries [F,W,Hq,S,E] (from queries [W,Hq,S,E] and full-width
 * cos/sin [F,W,S,R]) and then runs dvattn_sdpa on it.
 * Replaces binding.cu:356-372.  Same workspace size as dvattn_sdpa. */
DVATTN_API dvattn_status dvattn_fused(int dtype, void* out, void* rotated_queries, float scale,
                           const int* locations, const void* queries, const int* fragment_lengths,
                           const void* const* key_fragments, const void* const* value_fragments,
                           const int* fragment_tokens, const int* fragment_batch,
                           const float* cosines, const float* sines, const dvattn_shape* shape,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ---- standalone query rotation ---------------------------------------------
 * dvattn_rope: out [F,W,Hq,S,E] from queries [W,Hq,S,E], cos/sin [F,W,S,R].
 * Replaces binding.cu:41-77 + rope.cuh:54-65.
 * dvattn_varlen_rope: out [F,T,Hq,E] from queries [T,Hq,E], cos/sin [F,T,R/2].
 * Replaces binding.cu:205-247 + rope.cuh:102-114. */
DVATTN_API dvattn_status dvattn_rope(int dtype, void* out, const void* queries, const float* cosines,
                          const float* sines, const dvattn_shape* shape, void* stream);
DVATTN_API dvattn_status dvattn_varlen_rope(int dtype, void* out, const void* queries, const float* cosines,
                                 const float* sines, const dvattn_shape* shape, void* stream);

/* ---- K side of a decode step: rotate new keys, append K/V into pages --------
 * For every new token (w, s) with positions[w,s] = p >= 0, page
 * block_tables[w, p / block_size], row p % block_size:
 *   k_cache[page, row, h, :] = rope(keys[w, h, s, :], cosines[w, s, :], sines[w, s, :])
 *   v_cache[page, row, h, :] = values[w, h, s, :]
 * rope is the reference's apply_rotary_pos_emb (attention.py:82-88): dims e < R
 * take x*cos + rotate_half(x)*sin reading all R entries of the cos/sin row,
 * dims >= R are copied; each product and the sum are rounded to the promoted
 * dtype of (keys, cos) and the result to the storage type, exactly as PyTorch
 * evaluates it.  rope_dtype is DVATTN_F32 or dtype (the model dtype the
 * transformers rotary embedding returns).  Tokens whose position is negative
 * (masked), past the block_tables row or on a page outside [0, num_blocks) are
 * not written.  Uses shape fields W, Hkv, S, E, Ev, block_size,
 * max_blocks_per_seq, num_blocks, rotary_dim; positions [W,S] and block_tables
 * [W,max_blocks_per_seq] are contiguous int32; the other tensors are described
 * by element strides (last dim contiguous; cos/sin strides may be 0 to
 * broadcast one row, which makes this merge_caches' constant-offset
 * re-rotation, attention.py:245-251).  Keys/values must not overlap the cache
 * rows this call writes (they may live elsewhere in the cache allocations).
 * Replaces attention.py:304 (key rotation) + attention.py:141-152 (append to the
 * sequence's cache, transformers Cache.update). */
typedef struct dvattn_kv_layout {
    long long key_strides[3];     /* keys [W,Hkv,S,E]: strides of w, h, s */
    long long value_strides[3];   /* values [W,Hkv,S,Ev] */
    long long rope_strides[2];    /* cosines / sines [W,S,R]: strides of w, s */
    long long k_cache_strides[3]; /* k_cache [num_blocks,block_size,Hkv,E]: page, row, head */
    long long v_cache_strides[3]; /* v_cache [num_blocks,block_size,Hkv,Ev] */
} dvattn_kv_layout;

DVATTN_API dvattn_status dvattn_paged_kv_append(int dtype, int rope_dtype, void* k_cache, void* v_cache,
                                     const int* block_tables, const int* positions, const void* keys,
                                     const void* values, const void* cosines, const void* sines,
                                     const dvattn_shape* shape, const dvattn_kv_layout* layout, void* stream);

/* ---- per-view locations and rotary cos/sin on the device ---------------------
 * locations [F,W,S] i32, cosines/sines [F,W,S,R] f32 (R = rotary_dim, full
 * width, both halves equal) from fragment_lengths [F] i32 (device; lengths
 * already including the S new tokens), order [W,F] i32 (order[w, j]: the view
 * index of sequence w's j-th segment, its own segment last) and inv_freq
 * [R/2] f32 (the model's rotary inverse frequencies):
 *   locations[f,w,s] = (sum of the lengths of w's segments from f's place in
 *                       its order to the end) - S + s
 *   cos/sin[f,w,s,i] = cos/sin(float(locations[f,w,s]) * inv_freq[i % (R/2)])
 *                      * attention_scaling
 * A view missing from a sequence's order gets location -1 and cos 1, sin 0.
 * round_dtype (-1, DVATTN_F16 or DVATTN_BF16) rounds cos/sin through that type,
 * as the reference does when the model runs in it (rotary output in the model
 * dtype, then .to(float)).
 * Replaces attention.py:158-186 (DVAttnCache.update's host loops and the
 * transformers rotary embedding call). */
DVATTN_API dvattn_status dvattn_view_metadata(int* locations, float* cosines, float* sines,
                                   const int* fragment_lengths, const int* order, const float* inv_freq,
                                   float attention_scaling, int round_dtype, int F, int W, int S,
                                   int rotary_dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DVATTN_AMD_H */
