/* lema_hip.h -- C ABI of liblema_hip.so, the MI355X (gfx950) kernels of Latest Exact Match
 * Attention's hot path.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers unless stated otherwise; the library never allocates,
 *     frees or synchronises. Work is enqueued on `stream` (a hipStream_t, NULL = the null
 *     stream), so every call can be captured into a HIP graph.
 *   - Sizes and strides are int64 and counted in ELEMENTS of the tensor they describe.
 *   - Codes are unsigned integers of `code_bytes` bytes (4 or 8). A reference int64 code is the
 *     same 64-bit pattern (code_bytes = 8); only equality is ever used.
 *   - Return value: LEMA_OK, or an error status whose message lema_last_error() returns
 *     (thread-local, valid until the next call on that thread).
 *
 * Citations are file:line in moritzbroe/latest_exact_match_attention.
 */
#ifndef LEMA_HIP_H
#define LEMA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum lema_status {
  LEMA_OK = 0,
  LEMA_TABLE_FULL = 1, /* the store could not place a key (code/lema/csrc/store.cpp:159-160) */
  LEMA_BAD_ARG = 2,    /* shapes, strides, alignment or sizes the kernels do not accept */
  LEMA_HIP_ERROR = 3   /* a HIP runtime call failed (launch, attribute query) */
};

enum lema_dtype { LEMA_F32 = 0, LEMA_F16 = 1, LEMA_BF16 = 2 };

/* How a query without a match is filled (code/lema/attention.py:157-158 vs store.cpp:92). */
enum lema_miss { LEMA_MISS_DENSE = 0, /* v[b, h, 0, :] * 0: a signed zero, NaN for inf/NaN */
                 LEMA_MISS_ZERO = 1 /* +0 bytes, the store path */ };

const char* lema_last_error(void);
/* The version of this C ABI (1). No counterpart in the reference. */
int lema_abi_version(void);

/* dst[0, bytes) = src[0, bytes) on the device (bytes a multiple of 16, both pointers 16-byte
 * aligned). No counterpart in the reference: the benchmark's roofline compares the kernels'
 * HBM rates with this copy's, the streaming rate the memory reaches in practice. */
int lema_device_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* Sign-pack projected queries or keys into one code per row.
 * Replaces pack_codes, code/lema/attention.py:82-97: bit j of the code of row (b, h, t) is
 * (z[b, h, t, j] >= 0) compared as a float (so -0.0 -> 1, NaN -> 0); LSB = dim 0.
 *   z      [B, H, T, D] of `dtype`, element strides (z_sb, z_sh, z_st), last dim contiguous
 *   D      1..64; code_bytes 4 requires D <= 32
 *   codes  contiguous [B, H, T] of code_bytes                                            */
int lema_pack_codes(const void* z, int32_t dtype, int64_t B, int64_t H, int64_t T, int32_t D,
                    int64_t z_sb, int64_t z_sh, int64_t z_st, void* codes, int32_t code_bytes,
                    void* stream);

/* For each of N rows of T positions: src[n, i] = the largest j < i with
 * kc[n, j] == qc[n, i], else -1.
 * Replaces latest_prev_match, code/lema/attention.py:100-132 (the reference returns int64).
 *   qc, kc  contiguous [N, T] codes of code_bytes
 *   src     contiguous [N, T] of src_bytes (4 = int32, 8 = int64)                       */
int lema_latest_prev_match(const void* qc, const void* kc, int32_t code_bytes, int64_t N,
                           int64_t T, void* src, int32_t src_bytes, void* stream);

/* The exact LEMA op without a store, resolve and gather fused in one kernel:
 * y[b, h, i, :] = v[b, h, src, :] with src as above, a miss filled per `miss`.
 * Replaces lema_hard(q, k, v) after pack_codes, code/lema/attention.py:155-158.
 *   qc, kc  contiguous [B*H, T] codes
 *   v       [B, H, T, dv] of `dtype`, element strides (v_sb, v_sh, v_st), last dim contiguous
 *   y       [B, H, T, dv] of `dtype`, element strides (y_sb, y_sh, y_st), last dim contiguous
 *   src     NULL, or contiguous [B*H, T] of src_bytes receiving the match indices        */
int lema_hard(const void* qc, const void* kc, int32_t code_bytes, const void* v,
              int32_t dtype, int64_t B, int64_t H, int64_t T, int64_t dv, int64_t v_sb,
              int64_t v_sh, int64_t v_st, void* y, int64_t y_sb, int64_t y_sh, int64_t y_st,
              int32_t miss, void* src, int32_t src_bytes, void* stream);

/* Workspace bytes lema_latest_prev_match_ws and lema_hard_ws use for N rows of T positions:
 * 8 KB per 1024 positions, 0 for rows of fewer than 64,513 positions (64 chunks of 1024;
 * shorter rows keep the backward scan, which is faster there, and need none). No reference counterpart: the reference's sort needs no scratch the
 * caller provides. */
int64_t lema_resolve_workspace_bytes(int64_t N, int64_t T);

/* lema_latest_prev_match and lema_hard with a workspace (256-byte aligned, at least
 * lema_resolve_workspace_bytes(N or B*H, T) bytes; NULL when that is 0): a first kernel writes
 * per chunk of 1024 keys a summary table (latest position per distinct code), and the
 * resolver looks keys before a chunk up there instead of scanning all of them. Same results,
 * same reference functions replaced (code/lema/attention.py:100-132, 155-158). */
int lema_latest_prev_match_ws(const void* qc, const void* kc, int32_t code_bytes, int64_t N,
                              int64_t T, void* src, int32_t src_bytes, void* workspace,
                              int64_t workspace_bytes, void* stream);
int lema_hard_ws(const void* qc, const void* kc, int32_t code_bytes, const void* v,
                 int32_t dtype, int64_t B, int64_t H, int64_t T, int64_t dv, int64_t v_sb,
                 int64_t v_sh, int64_t v_st, void* y, int64_t y_sb, int64_t y_sh, int64_t y_st,
                 int32_t miss, void* src, int32_t src_bytes, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* The gather alone, for given indices: y = v[src] (miss per `miss`).
 * Replaces code/lema/attention.py:157-158. Shapes and strides as in lema_hard;
 * src is contiguous [B*H, T] of src_bytes, every entry in [-1, T).                      */
int lema_gather(const void* v, int32_t dtype, int64_t B, int64_t H, int64_t T, int64_t dv,
                int64_t v_sb, int64_t v_sh, int64_t v_st, const void* src, int32_t src_bytes,
                void* y, int64_t y_sb, int64_t y_sh, int64_t y_st, int32_t miss,
                void* stream);

/* One exchange against the shared open-addressing store in device memory.
 * Replaces store_exchange, code/lema/csrc/store.cpp:122-162 (bound as lema_store.exchange,
 * store.cpp:164-167, called from HashStore.exchange, code/lema/cache.py:184-201).
 *   table   [cap, 16 + vbytes] bytes, the reference's slot format ([code u64 | state u64 |
 *           value]); all zeros = empty
 *   items   i in [0, n): position i % T of partition i / T, group g0 + i / T; in position
 *           order per partition: out[i] = value of (group, qc[i]) or zeros, then
 *           (group, kc[i]) -> values[i], latest write wins
 *   qc      n codes of code_bytes, or NULL to only insert (then out may be NULL)
 *   values, out  [n, vbytes] bytes; vbytes % 8 == 0
 *   counts  int64 per group: += newly claimed slots
 *   full    int32 flag set to 1 when some key found no free slot (the reference raises
 *           "hash table full" after such a pass; the caller checks the flag)             */
int lema_store_exchange(void* table, int64_t cap, int64_t vbytes, const void* qc, const void* kc,
                        int32_t code_bytes, const void* values, void* out, int64_t n, int64_t T,
                        int64_t g0, int64_t* counts, int32_t* full, void* stream);

/* Workspace bytes lema_store_exchange_ws needs for a call of n items, T positions per
 * partition and code_bytes codes; 0 when such a call does not use one: T <= 1024, or
 * T <= 2048 with more than 128 partitions (the chunked path is the faster one there). No reference counterpart: lema_store_exchange's long calls made
 * parallel. */
int64_t lema_store_workspace_bytes(int64_t n, int64_t T, int32_t code_bytes);

/* lema_store_exchange with a device workspace (256-byte aligned, at least
 * lema_store_workspace_bytes): a call for which that is non-zero then runs in sub-calls of
 * up to 32768 positions, each as a few kernels over all of its items (in-chunk resolution,
 * per-chunk key summaries and a scratch table of every (partition, code) of the sub-call),
 * instead of one launch per 1024 positions. Same results as lema_store_exchange
 * (code/lema/csrc/store.cpp:122-162). workspace NULL = lema_store_exchange. */
int lema_store_exchange_ws(void* table, int64_t cap, int64_t vbytes, const void* qc,
                           const void* kc, int32_t code_bytes, const void* values, void* out,
                           int64_t n, int64_t T, int64_t g0, int64_t* counts, int32_t* full,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of the device scratch array behind lema_store_exchange_noalloc, per GPU. */
#define LEMA_NOALLOC_SCRATCH_BYTES (64LL * 1024 * 1024)

/* lema_store_exchange with no workspace argument that allocates nothing: a call that takes
 * the bulk path (as lema_store_workspace_bytes would report) runs on a scratch array inside
 * the library, LEMA_NOALLOC_SCRATCH_BYTES per GPU, in consecutive slices of its partitions
 * sized to fit it. The array is part of the library's code object: it is reserved on every GPU
 * where the library's kernels are loaded, whether or not this entry point is ever called, and
 * lasts for the life of the process. Same
 * results as lema_store_exchange_ws. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops). Make the first
 * call on a device outside graph capture (it looks the scratch's address up). Calls that
 * overlap on one GPU (two streams, two threads) race on the shared scratch; calls in one
 * stream's order do not. A call whose single partition needs more scratch than that is
 * rejected with LEMA_BAD_ARG (none can at present: a sub-call spans at most 32,768
 * positions, about 4.5 MB of scratch per partition). */
int lema_store_exchange_noalloc(void* table, int64_t cap, int64_t vbytes, const void* qc,
                                const void* kc, int32_t code_bytes, const void* values,
                                void* out, int64_t n, int64_t T, int64_t g0, int64_t* counts,
                                int32_t* full, void* stream);

/* ---- fused model segments (bf16), what the reference compiles with torch.compile ---- */

/* out = silu(gate) * up over n bf16 elements (n % 8 == 0, 16-byte aligned), the silu rounded
 * to bf16 first as in SwiGLU.forward, code/lema/model.py:85-94. */
int lema_swiglu_bf16(const void* gate, const void* up, void* out, int64_t n, void* stream);

/* Pre-norm of a block: x_out = x + d (d may be NULL: then x_out is unused), h_out =
 * x_out / sqrt(mean(x_out^2) + eps) * w, rows of D bf16 (D % 8 == 0, D <= 4096, 16-byte
 * aligned). Replaces the residual add and nn.RMSNorm of Block.forward,
 * code/lema/model.py:212-255. */
int lema_rmsnorm_bf16(const void* x, const void* d, const void* w, float eps, int64_t rows,
                      int64_t D, void* x_out, void* h_out, void* stream);

/* loss[r] = logsumexp(logits[r, :V]) - logits[r, target[r]] from bf16 logits (row stride ld,
 * V and ld multiples of 8, targets in [0, V)), fp32. Replaces the per-chunk
 * F.cross_entropy(logits.float()) of code/lema/train.py:131-152. */
int lema_cross_entropy_bf16(const void* logits, int64_t rows, int64_t V, int64_t ld,
                            const int64_t* target, float* loss, void* stream);

/* out[r * out_stride] = argmax of row r of bf16 values (V and the row stride ld multiples of
 * 8): the first index of the maximum, NaN above every number, as torch.argmax. Replaces the
 * greedy pick of code/lema/decode.py:71-93 (logits.argmax(-1)), written straight into a
 * token buffer. */
int lema_argmax_bf16(const void* x, int64_t rows, int64_t V, int64_t ld, int64_t* out,
                     int64_t out_stride, void* stream);

/* out row i = table row ids[i] of D bf16 (D % 8 == 0), zeros for an id outside [0, vocab):
 * the token embedding of a decode step (nn.Embedding, code/lema/model.py's tok_emb). */
int lema_embedding_bf16(const void* table, int64_t vocab, int64_t D, const int64_t* ids,
                        int64_t n, void* out, void* stream);

/* ---- decode-shaped products on the matrix cores (bf16, fp32 accumulation) ---- */

/* y[M, N] = x[M, K] . w[N, K]^T rounded to bf16, for 1 <= M <= 32 rows (a decode step's
 * tokens). K % 32 == 0; row strides ldx, ldw, ldy in elements (multiples of 8, pointers 16-byte
 * aligned). Replaces nn.Linear on those shapes (code/lema/model.py:168-179, 85-94). */
int lema_skinny_gemm_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream);

/* The query or key projection straight to codes: z = x . w^T (as above, N = H * d), and
 * codes[(b * H + h) * T + t] for row m = b * T + t gets bit j = (bf16(z[m, h * d + j]) >= 0).
 * Replaces project + pack_codes (code/lema/model.py:168-175, code/lema/attention.py:82-97) on
 * decode shapes; 16 * c must be a multiple of d for some c in 1..4 (d = 24: 48 columns). */
int lema_skinny_pack_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t M,
                          int64_t N, int64_t K, int32_t d, int64_t T, void* codes,
                          int32_t code_bytes, void* stream);

/* y = r + x . w^T: the product as in lema_skinny_gemm_bf16, rounded to bf16, then added to the
 * bf16 residual r [M, ldy] and rounded again (y may alias r). Replaces the MLP's down
 * projection and the residual add after it, x + mlp(h) (code/lema/model.py:229-232). */
int lema_skinny_gemm_add_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw,
                              const void* r, void* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, void* stream);

/* A layer's three projections in one launch: the query and key projections (wq, wk: Nqk rows
 * of H * d) straight to codes as in lema_skinny_pack_bf16, and the value projection (wv: Nv
 * rows) to v [M, Nv] bf16. All three weights share the row stride ldw. Replaces project +
 * pack_codes (code/lema/model.py:168-175, 224-227, code/lema/attention.py:82-97) on decode
 * shapes. */
int lema_skinny_qkv_bf16(const void* x, int64_t ldx, const void* wq, const void* wk,
                         const void* wv, int64_t ldw, int64_t M, int64_t Nqk, int64_t Nv,
                         int64_t K, int32_t d, int64_t T, void* qcodes, void* kcodes,
                         int32_t code_bytes, void* v, void* stream);

/* A prefill's query and key projections straight to codes: qcodes and kcodes [M / T, N / d, T]
 * (rows of x are M / T streams of T positions) of x [M, K] . wq^T and x . wk^T (wq, wk
 * [N, K] bf16, row strides ldx, ldw), bit j of a head's code = (bf16(z_j) >= 0), z never
 * stored. A persistent MFMA GEMM with the sign-pack in its epilogue. Replaces project +
 * pack_codes (code/lema/model.py:168-175, code/lema/attention.py:82-97) on prefill shapes:
 * M a multiple of 2048, N a multiple of 256 up to 65536, K a multiple of 64, d a multiple of
 * 8 up to 64, code_bytes 4 for d <= 32 and 8 above, under 2 GiB of codes per projection
 * (M * N / d * code_bytes < 2^31). */
int lema_qk_pack_bf16(const void* x, int64_t ldx, const void* wq, const void* wk, int64_t ldw,
                      int64_t M, int64_t N, int64_t K, int32_t d, int64_t T, void* qcodes,
                      void* kcodes, int32_t code_bytes, void* stream);

/* out[M, N] = bf16(bf16(silu(g)) * u), g = bf16(x . wg^T), u = bf16(x . wu^T): the gate and
 * up projections and SwiGLU's product in one launch (code/lema/model.py:85-94), out row stride
 * N. */
int lema_skinny_swiglu_bf16(const void* x, int64_t ldx, const void* wg, const void* wu,
                            int64_t ldw, int64_t M, int64_t N, int64_t K, void* out,
                            void* stream);

/* The MLP input of a decode step and its gate and up products in one launch
 * (code/lema/model.py:229-232, 85-94): s = x + d (each sum rounded to bf16; d NULL: s = x),
 * h = bf16(s * rsqrt(mean(s^2) + eps) * nw) rounded exactly as lema_rmsnorm_bf16 rounds it,
 * and out = lema_skinny_swiglu_bf16 of h; x_out receives s when d is given (a buffer apart
 * from x and d). x, d, x_out: [M, K] bf16 rows, 16-byte aligned; M <= 32, K <= 2048, and
 * M * (K + 8) * 2 bytes plus the partial sums within a workgroup's 160 KB of LDS. */
int lema_skinny_norm_swiglu_bf16(const void* x, const void* d, const void* nw, float eps,
                                 void* x_out, const void* wg, const void* wu, int64_t ldw,
                                 int64_t M, int64_t N, int64_t K, void* out, void* stream);

/* The attention input of a decode step and its q, k and v projections in one launch
 * (code/lema/model.py:224-227, 168-175): h = bf16(x * rsqrt(mean(x^2) + eps) * nw) rounded
 * exactly as lema_rmsnorm_bf16 rounds it, then lema_skinny_qkv_bf16 of h (rows of K). x:
 * [M, K] bf16 rows, 16-byte aligned; M <= 32, K <= 2048, and M * (K + 8) * 2 bytes plus the
 * partial sums within a workgroup's 160 KB of LDS. Replaces norm1 + project + pack_codes. */
int lema_skinny_norm_qkv_bf16(const void* x, const void* nw, float eps, const void* wq,
                              const void* wk, const void* wv, int64_t ldw, int64_t M,
                              int64_t Nqk, int64_t Nv, int64_t K, int32_t d, int64_t T,
                              void* qcodes, void* kcodes, int32_t code_bytes, void* v,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LEMA_HIP_H */
