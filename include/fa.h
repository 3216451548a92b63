/*
 * fa.h - C ABI of libfa.so, the MI355X (gfx950) fused causal attention library.
 *
 * Every entry point enqueues work on the caller's HIP stream and returns
 * without synchronising.  The caller owns every buffer (inputs, outputs, LSE
 * and the backward's workspace); no call allocates device memory, and none
 * keeps a pointer after it returns.  The library does hold one static device
 * array: the 64 MiB scratch behind fa_bwd_gqa_noalloc, which every device the
 * loaded library runs on carries (in its code object's memory) until the
 * process ends, whichever entry points a caller uses.  All tensors are dense,
 * row-major [B, heads, S, D] in device memory; LSE is dense [B, H, S] float32.
 *
 * Return value: FA_OK (0) or one of the negative FA_ERR_* codes below.
 * fa_strerror() turns a code into a static message.
 */
#ifndef FA_H
#define FA_H

#if defined(__GNUC__) || defined(__clang__)
#define FA_API __attribute__((visibility("default")))
#else
#define FA_API
#endif

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fa_dtype { FA_F16 = 0, FA_BF16 = 1 };

enum fa_status {
  FA_OK = 0,
  FA_ERR_DIMS = -1,     /* B, H, H_kv or S not positive, H % H_kv != 0, or
                           B*H*S or S*D*2 (bytes of one head's rows) >= 2^31 */
  FA_ERR_DTYPE = -2,    /* dtype is neither FA_F16 nor FA_BF16 */
  FA_ERR_HEADDIM = -3,  /* D not in {32, 64, 128} */
  FA_ERR_TILE = -4,     /* block_m / block_n not in {64, 128} */
  FA_ERR_NULL = -5,     /* a required pointer is NULL */
  FA_ERR_LAUNCH = -6,   /* the HIP runtime rejected a launch */
  FA_ERR_UNSUPPORTED = -7, /* valid arguments, but no kernel for this combination */
  FA_ERR_WORKSPACE = -8,   /* fa_bwd_gqa*: workspace not 16-byte aligned; fa_bwd_gqa_exact:
                              also a workspace too small for the requested split */
  FA_ERR_SCRATCH = -9      /* fa_bwd_gqa_noalloc: the per-row terms exceed the library's scratch */
};

/*
 * Causal forward O = softmax(Q K^T / sqrt(D) + causal mask) V, optionally
 * writing the per-row log-sum-exp.
 *
 * Replaces the device launch of:
 *   attention/fused/fused.py:68-76        fused_attention          (H_kv == H, lse NULL)
 *   attention/gqa/fused_gqa.py:70-82      fused_gqa_attention      (H_kv divides H, lse NULL)
 *   attention/backward/fused_backward.py:161-170  _forward         (H_kv == H, lse non-NULL)
 *
 * q, o : [B, H, S, D]      k, v : [B, H_kv, S, D]     element type = dtype
 * lse  : NULL, or [B, H, S] float32 receiving m + log2(l): the base-2 log-sum-exp
 *        of the scores pre-multiplied by scale_log2 (the quantity the reference
 *        builds at attention/backward/fused_backward.py:169).
 * scale_log2 : log2(e) / sqrt(D) as the reference folds it (fused.py:74).
 * Query head h reads K/V head h / (H / H_kv) (fused_gqa.py:18).
 * block_m / block_n : query rows per head and keys per LDS tile, each in {64, 128}.
 *        block_m cannot change the result (each 32-row wave computes the same
 *        either way); where a 64-row single-head workgroup would leave SIMDs idle
 *        the library runs 128-row workgroups.
 *        S may be any length >= 1: a partial last query or key tile is masked (the
 *        reference requires S to be a multiple of both tiles, fused.py:70-71, and
 *        names partial edge tiles as future work).
 */
FA_API int fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
           int B, int H, int H_kv, int S, int D, int dtype, float scale_log2,
           int block_m, int block_n, void* hip_stream);

/*
 * Recompute backward of the causal forward: dQ, dK, dV from Q, K, V, O, dO and
 * the LSE written by fa_fwd.  Atomic-free kernels run in order on the stream: a
 * row pass writes -LSE/c and -Delta (Delta = rowsum(dO * O)) of every query row
 * into the start of dq's own buffer (8 bytes of each row's 2 D bytes), dK/dV (one
 * workgroup per key tile) reads them, then dQ (one workgroup per query tile) forms
 * its own and overwrites dq.  No workspace.  When dq is not 16-byte aligned the
 * dK/dV kernel forms Delta from the O and dO tiles of every key tile instead (same
 * results up to the fp32 summation order of Delta, slower).
 *
 * Replaces attention/backward/fused_backward.py:173-184 (_backward: the torch
 * Delta op at :175 and the two launches at :180-183).
 *
 * q, k, v, o, d_o, dq, dk, dv : [B, H, S, D] (MHA, as the reference's _check
 * requires at fused_backward.py:154); lse : [B, H, S] float32 from fa_fwd.
 * sm_scale = 1/sqrt(D) scales dQ and dK once at the end (fused_backward.py:105,146).
 */
FA_API int fa_bwd(const void* q, const void* k, const void* v, const void* o,
           const void* d_o, const float* lse, void* dq, void* dk, void* dv,
           int B, int H, int S, int D, int dtype, float scale_log2, float sm_scale,
           int block_m, int block_n, void* hip_stream);

/*
 * The same backward for grouped-query attention: q, o, d_o, dq are [B, H, S, D],
 * k, v, dk, dv are [B, H_kv, S, D] with H_kv dividing H, lse is [B, H, S] from
 * fa_fwd; query head h reads K/V head h / (H / H_kv).  dK and dV of a K/V head
 * are the sums over its H / H_kv query heads, without atomics.
 *
 * workspace: NULL, or caller-owned device memory of workspace_bytes bytes,
 * 16-byte aligned, used in two parts, each only if the rest of the workspace
 * holds it:
 *  1. 8 * B * H * S bytes (rounded up to 256): -LSE/c and -Delta of every query
 *     row.  The dQ kernel then runs first and writes them, and the dK/dV kernel
 *     reads them instead of forming Delta from the O and dO tiles in each of the
 *     key tiles that meet a query tile (about 10 % of its time at S = 4096).
 *  2. fp32 partial dK/dV.  Without them one workgroup per 128-key tile walks every
 *     (query tile, query head) pair of the tile and sums them in registers, which
 *     leaves most of the GPU idle when B * H_kv * S / 128 is small (MQA, few heads,
 *     small batch).  With them each key tile's pairs are split over several
 *     workgroups that write fp32 partial sums, and a reduction pass on the same
 *     stream adds them up (fixed order, deterministic); a smaller remainder gets
 *     the largest split it holds.
 * fa_bwd_gqa_workspace_size() gives the bytes for both.  The workspace must stay
 * allocated until the stream has passed this call.  H_kv = H (MHA) is accepted:
 * that is how an MHA caller gets either.
 *
 * No counterpart in the reference, whose backward is MHA-only (_check at
 * attention/backward/fused_backward.py:154 rejects K/V of another head count);
 * fa_bwd(...) equals fa_bwd_gqa(..., H_kv = H, ..., NULL, 0, stream).  Without a
 * workspace (or with one too small for the per-row terms) the row pass of fa_bwd
 * keeps them in dq's buffer, with the same results as when the workspace holds them.
 */
FA_API int fa_bwd_gqa(const void* q, const void* k, const void* v, const void* o,
               const void* d_o, const float* lse, void* dq, void* dk, void* dv,
               int B, int H, int H_kv, int S, int D, int dtype, float scale_log2, float sm_scale,
               int block_m, int block_n, void* workspace, size_t workspace_bytes, void* hip_stream);

/*
 * fa_bwd_gqa for callers that cannot allocate device memory -- code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc.  No counterpart in the
 * reference.  Same arguments as fa_bwd_gqa, and the results of
 * fa_bwd_gqa(..., workspace, fa_noalloc_scratch_bytes(), stream) bitwise: the workspace
 * is the library's own device scratch, a static array of fa_noalloc_scratch_bytes() =
 * 64 MiB that each device holds from the library's first use on it until the process
 * ends.  The per-row terms come first; the dK/dV split is the one the shape asks for
 * when its partial sums fit behind them, else the largest that fits (possibly none).
 * The call allocates nothing (no hipMalloc, no hipFree, no allocating library routine).
 *   Limit: shapes whose per-row terms (8 * B * H * S bytes, i.e. B * H * S above 8M
 *   rows) exceed 64 MiB are rejected with FA_ERR_SCRATCH before anything is enqueued.
 *   Every call on a device shares that device's scratch: calls whose work overlaps on
 *   one device (different streams, or host threads without ordering) race; serialise
 *   them on one stream.  Nothing in the scratch needs to start at zero.
 */
FA_API int fa_bwd_gqa_noalloc(const void* q, const void* k, const void* v, const void* o,
                       const void* d_o, const float* lse, void* dq, void* dk, void* dv,
                       int B, int H, int H_kv, int S, int D, int dtype, float scale_log2, float sm_scale,
                       int block_m, int block_n, void* hip_stream);

/* Bytes of the device scratch behind fa_bwd_gqa_noalloc (per device).  No reference
 * counterpart. */
FA_API size_t fa_noalloc_scratch_bytes(void);

/*
 * Tile and occupancy studies.  The entry points above pick the workgroup shape by
 * rules (rows per workgroup, heads per workgroup, dK/dV split); these run the shape
 * that is asked for, literally, so each rule's rejected variants can be measured
 * beside its choice (the reference measures every tile as requested:
 * profiling/3_tile_study/README.md:8-19).  No counterpart in the reference's API.
 *
 * fa_fwd_exact: fa_fwd with block_m query rows per head and heads_per_wg query heads
 *   (of one K/V group) per workgroup, block_n keys per tile.  FA_ERR_UNSUPPORTED when no
 *   kernel has that shape ((block_m, block_n, heads_per_wg) in {64,128}x{64,128}x{1},
 *   {64,128}x{64}x{2}, (64,128,2), (64,64,4)).
 * fa_bwd_gqa_exact: fa_bwd_gqa with the dQ kernel at dq_block_m x dq_block_n and the
 *   dK/dV key tiles split nsplit ways (1..64; > 1 needs a workspace of
 *   8*B*H*S (rounded up to 256) + 8*B*H_kv*nsplit*S*D bytes, else FA_ERR_WORKSPACE).
 *   A NULL workspace (nsplit 1) runs the dK/dV kernel that forms Delta in every key
 *   tile it meets, then dQ: the variant the row terms replace, kept for measurement.
 * The queries return what fa_fwd / fa_bwd_gqa choose for a shape (0: invalid).
 */
FA_API int fa_fwd_exact(const void* q, const void* k, const void* v, void* o, float* lse,
                 int B, int H, int H_kv, int S, int D, int dtype, float scale_log2,
                 int block_m, int block_n, int heads_per_wg, void* hip_stream);
FA_API int fa_bwd_gqa_exact(const void* q, const void* k, const void* v, const void* o,
                     const void* d_o, const float* lse, void* dq, void* dk, void* dv,
                     int B, int H, int H_kv, int S, int D, int dtype, float scale_log2, float sm_scale,
                     int dq_block_m, int dq_block_n, int nsplit, void* workspace, size_t workspace_bytes,
                     void* hip_stream);
FA_API int fa_fwd_heads_per_wg(int B, int H, int H_kv, int S, int D, int block_m, int block_n);
FA_API int fa_fwd_rows_per_wg(int block_m, int block_n, int D, int heads_per_wg);
FA_API int fa_bwd_dq_rows_per_wg(int block_m, int D);
FA_API int fa_bwd_dkdv_split(int B, int H, int H_kv, int S, int D);

/* Workspace bytes fa_bwd_gqa uses for this shape on the current device: the
 * per-row terms, plus the partial sums when the key tiles alone leave the GPU
 * idle (0 for invalid dimensions).  No reference counterpart. */
FA_API size_t fa_bwd_gqa_workspace_size(int B, int H, int H_kv, int S, int D);

/* 1 if a forward (with_lse 0/1) or backward (is_bwd 1) kernel exists for the
 * combination, else 0.  No reference counterpart: it lets a caller probe the
 * supported (dtype, D, tile) set before validating inputs. */
FA_API int fa_supported(int dtype, int D, int block_m, int block_n, int group, int with_lse, int is_bwd);

/* Static, NUL-terminated description of a status code. */
FA_API const char* fa_strerror(int status);

/* Library version as 10000*major + 100*minor + patch. */
FA_API int fa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA_H */
