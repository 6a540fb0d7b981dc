/*
 * detllm_hip.h — C ABI of libdetllm_hip.so, the MI355X (gfx950) "rocm"
 * backend of DetLLM's integer forward pass.
 *
 * Conventions (every entry point):
 *   - pointers are DEVICE pointers owned by the caller (torch allocator);
 *     nothing is allocated, freed, synchronised or read back on the host,
 *     so every call is safe inside hipGraph stream capture;
 *   - shapes are explicit ints, arrays are dense row-major;
 *   - work is enqueued on the given hipStream_t;
 *   - return 0 on success, > 0 = hipError_t of a failed launch,
 *     < 0 = argument error (-22 EINVAL, -34 ERANGE, -38 ENOSYS).
 *   - every result is an integer bit-identical to the reference CPU
 *     ("reference") backend: int64 wraps, torch shift clamping, floor
 *     division, round_half_away_div / rshift_round rounding
 *     (src/detllm/intmath.py:7-17). Inputs, outputs and stored state are
 *     integers; inside some kernels a quotient is obtained as the truncation
 *     of a biased fp64 (or fp32) estimate that provably equals the exact
 *     integer under operand bounds each kernel checks, else the integer
 *     routine runs (csrc/intops.h states each bound; the library refuses to
 *     build under -ffast-math);
 *   - err (where present, nullable) is a device int32 word: an index the
 *     reference would reject with IndexError sets bit 1 (token id outside
 *     [-vocab, vocab)), bit 2 (position outside [-max_pos, max_pos)), and a
 *     device slot count above a launch's slot bound bit 4; the kernel then
 *     reads row 0 / scans the bounded slots, and the host raises from the
 *     word at its next check (negative indices wrap as in torch).
 *
 * Reference interfaces each entry replaces are cited as file:line in
 * rishabh135/idempotent_llm. The reference has no FFI: its boundary is the
 * Python function named in each citation; the Python mirror in
 * idempotent_llm_amd/ binds these symbols through ctypes.
 */
#ifndef DETLLM_HIP_H
#define DETLLM_HIP_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- GEMM -- */

/* int_gemm(a, b, backend) — src/detllm/backends.py:88-135 (batched form
 * :127-134). C[b] = A[b] . B[b]^T: A [batch][M][K], B [batch][N][K] (the
 * artifact's [K][N] w8t transposed), C [batch][M][N] int32; batch strides in
 * elements. K % 16 == 0, K <= 131071. i8 MFMA: 32x32x32 tiles of 256x256,
 * 128x192, 128x128 or 128x64 elements per block by tile count when K % 128
 * == 0 (a direct-to-LDS operand ring), else 128x128 blocks of 16x16x64. */
int detllm_igemm_nt(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K,
                    int batch, int64_t sA, int64_t sB, int64_t sC, hipStream_t s);

/* int_gemm for M <= 64 (decode GEMV) — backends.py:88-135 (2-D path :115-119,
 * decode fast path :121-126). Writes ksplit int32 partials C[k][M][N],
 * split_stride elements apart, whose integer sum is the product (ksplit = 1:
 * the product itself). */
int detllm_igemv_nt(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K,
                    int ksplit, int64_t split_stride, hipStream_t s);

/* detllm_igemv_nt plus a prefetch hint (no counterpart in the reference: a
 * performance hint of this backend): up to four device byte ranges
 * (pf_i, n_i; n_i a multiple of 4, 0 = unused) that the following kernels
 * read are touched once per 128-byte line while the weights stream, so they
 * sit in the memory-side cache when those kernels start. Results are those
 * of detllm_igemv_nt. */
int detllm_igemv_nt_pf(const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K,
                       int ksplit, int64_t split_stride, const void* pf0, int64_t n0,
                       const void* pf1, int64_t n1, const void* pf2, int64_t n2,
                       const void* pf3, int64_t n3, hipStream_t s);

/* K split that detllm_igemv_nt is tuned for at this shape (the reference's
 * cuBLASLt path picks its own kernel internally, backends.py:115-119);
 * writes *ksplit in [1, 8]. */
int detllm_igemv_plan(int M, int N, int K, int* ksplit);

/* Device transpose of int8 [R][C] matrices (operand layout for int_gemm's
 * [K][N] right-hand side; backends.py:115-119 consumes b as [K][N]). */
int detllm_transpose_i8(const int8_t* src, int8_t* dst, int R, int C, int batch,
                        int64_t sS, int64_t sD, hipStream_t s);

/* IntQwen3.greedy_pick — src/detllm/model.py:482-490: out[r] = lowest v
 * maximising logits[r][v] * head_m[v] (int64). pv/pi: R * ceil(V/chunk)
 * int64 scratch each. */
int detllm_greedy_pick(const int32_t* logits, const int64_t* head_m, int R, int V, int chunk,
                       int64_t* pv, int64_t* pi, int64_t* out, hipStream_t s);

/* No counterpart in the reference: detllm_greedy_pick for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same result as detllm_greedy_pick with
 * chunk 2048; the partials live in the library's own per-device scratch
 * array (2 x 32768 int64 = 512 KiB per GPU, held until the process ends), so
 * R * ceil(V / 2048) <= 32768 or the call returns -34 (ERANGE). The first
 * call on a device resolves that device's array address (do it outside
 * capture). Calls that overlap on one GPU share the array and race; the
 * caller orders them (one stream, or events). Allocates nothing. */
int detllm_greedy_pick_noalloc(const int32_t* logits, const int64_t* head_m, int R, int V,
                               int64_t* out, hipStream_t s);

/* Compact digest of logits rows for the determinism harness (scripts/demo.py:
 * 58-75 hashes whole rows on the host; this 64-bit digest lets rows be
 * compared on the device): out[r] = sum over v of splitmix64_mix((v << 32) |
 * (uint32) logits[r][v]) modulo 2^64, as int64. */
int detllm_logits_digest(const int32_t* logits, int R, int V, int64_t* out, hipStream_t s);

/* ------------------------------------------------- fused layer kernels -- */

/* Embedding lookup + residual_from_delta + _norm_quant —
 * model.py:246-249 (dyadic.py:187-190, :174-184) fused with model.py:187-198
 * for the first layer's attention input (sm_m = as_m of layer 0; null skips
 * the smoothing multiply; x8 null skips the norm-quant). h [R][C] int32,
 * k_res/xm/xk [R] int64, x8 [R][C] int8. Ids index as embed_e8[ids] does
 * (negative ids wrap); an id outside [-vocab, vocab) sets bit 1 of *err. */
int detllm_embed_normq(const int64_t* ids, int R, int C, int64_t vocab, const int8_t* e8,
                       const int64_t* em, const int64_t* ek, int32_t* h, int64_t* k_res,
                       const int64_t* sm_m, int64_t sm_k, int8_t* x8, int64_t* xm, int64_t* xk,
                       int32_t* err, hipStream_t s);

/* The next skinny GEMM (next_w, next_n, next_k, next_ksplit), the trailing
 * arguments of the three row kernels below: the product detllm_igemv_nt
 * computes right after this launch, W [next_n][next_k] int8 with that K
 * split. At decode sizes (R <= 64) the launch adds blocks that pull W's
 * slices into the L2 cache of the XCD whose GEMM blocks will read them. A
 * performance hint with no counterpart in the reference: results do not
 * depend on it; next_w null (and zeros) adds nothing.
 *
 * Deferred scale fit (the last argument before the stream). A producer of a
 * GEMM operand (detllm_swiglu_quant, detllm_merge_rowcol) with defer_fit =
 * 1 does not run the fit (m, e) = fit_dyadic_ratio(num, 127)
 * (dyadic.py:52-72) that ends quant_i8_pertoken / requant_i8_rowcol
 * (dyadic.py:104-105, :138-139): it stores num in place of m and the row's
 * k without e in place of k. The consumer of that GEMM's partials
 * (detllm_residual_normq with row_fit = 1) runs the fit, on every lane
 * while its partials are in flight, instead of the producer's one lane at
 * the end of its launch. The integers are the same either way. This is an
 * order of operations with no counterpart in the reference; 0 stores and
 * reads (m, k) as dyadic.py does. */

/* requant_i32_common(P, row_m, row_k, col_m, col_k, tb) + residual_add +
 * _norm_quant(sm_m, sm_k) — model.py:410-415 / :424-427, :303, :284
 * (dyadic.py:108-120, :193-206; ops/di_rmsnorm.py:33-52; dyadic.py:93-105).
 * P: nsplit int32 partials [nsplit][R][C]; h/k_res updated in place. */
int detllm_residual_normq(const int32_t* P, int nsplit, int64_t split_stride, int R, int C,
                          const int64_t* row_m, const int64_t* row_k, const int64_t* col_m,
                          int64_t col_k, int tb, int32_t* h, int64_t* k_res,
                          const int64_t* sm_m, int64_t sm_k, int8_t* x8, int64_t* xm,
                          int64_t* xk, const int8_t* next_w, int next_n, int next_k,
                          int next_ksplit, int row_fit, hipStream_t s);

/* Decode skinny GEMMs with the row kernel that makes their int8 operand
 * fused in (R <= 8 rows). Results equal the two launches they replace: the
 * row kernel below, then detllm_igemv_nt into C [ksplit][R][N] with the K
 * split of detllm_igemv_plan. Every block recomputes the operand rows (in
 * LDS, while its weight loads are in flight); one block stores the rows'
 * other outputs. Shapes outside the fused kernel's range return -38 (ENOSYS)
 * and the caller runs the two launches.
 *
 * detllm_igemv_resnormq: operand = detllm_residual_normq of (P, row_m, row_k,
 * col_m, col_k, tb) on the residual h_in / k_res_in — model.py:410-415,
 * :424-427, :187-198 — which it writes to h_out / k_res_out (h_out must not
 * alias h_in: other blocks still read it) and whose (m, k) go to xm / xk;
 * K <= 1024. W [N][K] the next product's weights. */
int detllm_igemv_resnormq(const int8_t* W, int32_t* C, int R, int N, int K, int ksplit,
                          int64_t split_stride, const int32_t* P, int nsplit,
                          int64_t p_split_stride, const int64_t* row_m, const int64_t* row_k,
                          const int64_t* col_m, int64_t col_k, int tb, const int32_t* h_in,
                          const int64_t* k_res_in, int32_t* h_out, int64_t* k_res_out,
                          const int64_t* sm_m, int64_t sm_k, int64_t* xm, int64_t* xk,
                          const void* pf0, int64_t n0, const void* pf1, int64_t n1,
                          hipStream_t s);

/* detllm_merge_rowcol of decode rows (one partial of attn [R][C], C <= 2048,
 * R <= 64) from the row statistics detllm_qkv_attn_decode_ext writes (ext
 * [R][n_ext][2], n_ext = n_kv <= 8): every value elementwise — the same
 * integers as requant_i8_rowcol (dyadic.py:123-139, model.py:404-409) — in
 * 256-column pieces, one block each. om [C]: the per-column product
 * os_m * col_m; the other arguments as detllm_merge_rowcol's. */
int detllm_merge_ext(const int64_t* attn, int R, int C, const int64_t* om, int64_t os_k,
                     int64_t col_k, const int64_t* ext, int n_ext, int8_t* a8, int64_t* am,
                     int64_t* ak, const int8_t* next_w, int next_n, int next_k, int next_ksplit,
                     int defer_fit, hipStream_t s);

/* detllm_igemv_merge_ext: detllm_igemv_merge (one partial of attn [R][K])
 * whose merge statistics come from ext [R][n_ext][2] as
 * detllm_qkv_attn_decode_ext writes them (n_ext = n_kv), so each block
 * quantises only its K range of the operand rows, every value elementwise —
 * the same integers as requant_i8_rowcol (dyadic.py:123-139, model.py:
 * 404-409). om [K]: the per-column product os_m * col_m; n_ext <= 8;
 * defer_fit as in detllm_merge_rowcol. */
int detllm_igemv_merge_ext(const int8_t* W, int32_t* C, int R, int N, int K, int ksplit,
                           int64_t split_stride, const int64_t* attn, const int64_t* om,
                           int64_t os_k, int64_t col_k, const int64_t* ext, int n_ext,
                           int64_t* am, int64_t* ak, int defer_fit, const void* pf0, int64_t n0,
                           const void* pf1, int64_t n1, hipStream_t s);

/* detllm_igemv_merge: operand = the attention-output merge
 * requant_i8_rowcol(attn * os_m, 1, os_k, col_m, col_k) — model.py:404-409 —
 * of int64 attn [nsplit][R][K], K <= 2048; col_m may be null when os_m holds
 * the per-column product os_m * col_m. (m, k) to am / ak. */
int detllm_igemv_merge(const int8_t* W, int32_t* C, int R, int N, int K, int ksplit,
                       int64_t split_stride, const int64_t* attn, int nsplit,
                       int64_t a_split_stride, const int64_t* os_m, int64_t os_k,
                       const int64_t* col_m, int64_t col_k, int64_t* am, int64_t* ak,
                       const void* pf0, int64_t n0, const void* pf1, int64_t n1, hipStream_t s);

/* detllm_igemv_swiglu: operand = detllm_swiglu_quant of ONE decode row's
 * gate|up product (P [nsplit][1][2K], p_split_stride apart) — model.py:416-423
 * (dyadic.py:108-120 twice, ops/di_swiglu.py:39-58, dyadic.py:93-105) — whose
 * row scale goes to ym / yk (fitted unless defer_fit, as detllm_swiglu_quant);
 * K = the intermediate size, a multiple of 512, at most 3072; W [N][K] the
 * down projection's weights. The int8 row itself stays in LDS. */
int detllm_igemv_swiglu(const int8_t* W, int32_t* C, int N, int K, int ksplit,
                        int64_t split_stride, const int32_t* P, int nsplit, int64_t p_split_stride,
                        const int64_t* xm, const int64_t* xk, const int64_t* gate_m,
                        int64_t gate_k, const int64_t* up_m, int64_t up_k, const int64_t* ds_m,
                        int64_t ds_k, int64_t* ym, int64_t* yk, int defer_fit, const void* pf0,
                        int64_t n0, const void* pf1, int64_t n1, hipStream_t s);

/* IntQwen3._norm_quant — model.py:187-198: di_rmsnorm(h) (ops/di_rmsnorm.py:33-52),
 * optional smoothing multiply by sm_m (null: none) with k 20 + sm_k, then
 * quant_i8_pertoken (dyadic.py:93-105). h [R][C] int32 is only read. */
int detllm_norm_quant(const int32_t* h, int R, int C, const int64_t* sm_m, int64_t sm_k,
                      int8_t* x8, int64_t* xm, int64_t* xk, hipStream_t s);

/* gate/up requant_i32_common(14) x2 + di_swiglu + quant_i8_pertoken(y*ds_m)
 * — model.py:416-423 (ops/di_swiglu.py:39-58). P: [nsplit][R][2I] with gate
 * in columns [0, I) and up in [I, 2I). */
int detllm_swiglu_quant(const int32_t* P, int nsplit, int64_t split_stride, int R, int I,
                        const int64_t* xm, const int64_t* xk, const int64_t* gate_m,
                        int64_t gate_k, const int64_t* up_m, int64_t up_k, const int64_t* ds_m,
                        int64_t ds_k, int8_t* y8, int64_t* ym, int64_t* yk,
                        const int8_t* next_w, int next_n, int next_k, int next_ksplit,
                        int defer_fit, hipStream_t s);

/* Attention-output merge: requant_i8_rowcol(attn * os_m, 1, os_k, col_m,
 * col_k) — model.py:404-409 (dyadic.py:123-139). attn: [nsplit][R][C] int64
 * partial context sums. */
int detllm_merge_rowcol(const int64_t* attn, int nsplit, int64_t split_stride, int R, int C,
                        const int64_t* os_m, int64_t os_k, const int64_t* col_m, int64_t col_k,
                        int8_t* a8, int64_t* am, int64_t* ak, const int8_t* next_w,
                        int next_n, int next_k, int next_ksplit, int defer_fit,
                        hipStream_t s);

/* The KV cache is paged. Per layer, a K pool [n_pages][n_kv][128][128] (a
 * page's K rows: n_kv heads x 128 slots x 128 channels) and a V pool
 * [n_pages][n_kv][128][128] (V transposed: channels x slots); table
 * [B][width] int32 gives row b's page for slots [128 j, 128 j + 128)
 * (-1: not mapped; such slots are never written and never read as data:
 * the kernels mask them, reading page 0's bytes in their place, so a pool
 * holds at least one page). A row holds width * 128 slots. The reference keeps one contiguous
 * [B, n_kv, CAP, hd] buffer per layer (model.py:67-102): same contents, only
 * the addressing differs, so pages allocated as a cache grows never move
 * earlier slots.
 *
 * Q/K/V epilogue per (token, head) — model.py:200-216 (_qk_head_pipeline),
 * :303-340 (QK smoothing, Q quant_i8_pertoken, K/V requant_i8_static, cache
 * write) and :351-358 (score scale norm_scale + DI-Exp constant tpos).
 * P: [nsplit][B*T][(n_q + 2 n_kv) * 128] int32 (q | k | v columns).
 * Outputs: q8 [B][n_q][T][128], tpos [B][n_q][T]; optional dbg
 * [B][n_q][T][4] = (qm, qk, sm, sk); K and V into the paged cache at slot
 * base + t, where base is *slot_base_dev when non-null (graph replay) else
 * slot_base. Positions
 * index the RoPE tables as cos_t[positions] does; one outside
 * [-max_pos, max_pos) sets bit 2 of *err. */
int detllm_qkv_epilogue(const int32_t* P, int nsplit, int64_t split_stride, int B, int T,
                        int n_q, int n_kv, const int64_t* xm, const int64_t* xk,
                        const int64_t* positions, const int64_t* q_m, int64_t q_k,
                        const int64_t* k_m, int64_t k_k, const int64_t* v_m, int64_t v_k,
                        const int64_t* q_norm_m, int64_t q_norm_k, const int64_t* k_norm_m,
                        int64_t k_norm_k, const int64_t* qs_m, int64_t qs_k,
                        const int64_t* kq_m, const int64_t* kq_k, const int64_t* ks_m,
                        const int64_t* ks_k, const int64_t* vq_m, const int64_t* vq_k,
                        const int16_t* cos_t, const int16_t* sin_t, int64_t max_pos,
                        int8_t* q8, int64_t* tpos, int64_t* dbg, int8_t* kpool,
                        int8_t* vpool, const int32_t* table, int width,
                        const int64_t* slot_base_dev, int64_t slot_base, const int64_t* kq_est,
                        int32_t* err, hipStream_t s);

/* The static K requantisation's per-channel divisors for one layer
 * (requant_i8_static of model.py:326-329 with row scale (1, rowk), rowk =
 * 20 + k_norm_k), computed once at model load: est [n][4] = {den = kq_m <<
 * max(rowk - kq_k, 0) (wrapping; 1 if 0), up = max(kq_k - rowk, 0), the bits
 * of fl(1/den) and of fl((floor(den/2) + 1/2) / den)}. detllm_qkv_epilogue
 * reads them through kq_est (nullable: then it derives them per element). */
int detllm_kq_est(const int64_t* kq_m, const int64_t* kq_k, int64_t n, int64_t rowk,
                  int64_t* est, hipStream_t s);

/* requant_i8_static of a GEMM output — src/detllm/dyadic.py:142-163 with
 * per-row (row_m, row_k) (null: (1, 0)), per-column col_m [C], scalar col_k
 * and a scalar static target (s_m, s_k): y8 = clamp_i8(rhad(P col_m row_m
 * << up, s_m << down)), shift = row_k + col_k - s_k. P: nsplit int32
 * partials [nsplit][R][C]. Config c0's epilogue is (P, 1, 0, m, 20, 1, 0). */
int detllm_requant_static_cols(const int32_t* P, int nsplit, int64_t split_stride, int R, int C,
                               const int64_t* row_m, const int64_t* row_k, const int64_t* col_m,
                               int64_t col_k, int64_t s_m, int64_t s_k, int8_t* y8,
                               hipStream_t s);

/* int_gemm followed by requant_i8_static, for M <= 64 rows, in one launch —
 * src/detllm/backends.py:88-135 then dyadic.py:142-163 (config c0: A int8
 * [64][1024] x the [1024][3072] weight, (P, 1, 0, m, 20, 1, 0)). A [M][K], B
 * [N][K] (the weight transposed, as detllm_igemv_nt takes it); the int32
 * product stays in registers and y8 [M][N] = clamp_i8(rhad(P col_m row_m <<
 * up, s_m << down)), shift = row_k + col_k - s_k; row_m / row_k nullable (1,
 * 0). Same integers as detllm_igemv_nt + detllm_requant_static_cols.
 * K % 16 == 0, K <= 131071. */
int detllm_igemv_requant_static(const int8_t* A, const int8_t* B, int M, int N, int K,
                                const int64_t* row_m, const int64_t* row_k,
                                const int64_t* col_m, int64_t col_k, int64_t s_m, int64_t s_k,
                                int8_t* y8, hipStream_t s);

/* ------------------------------------------------------------ attention -- */

/* Prefill/chunk attention — model.py:382-402 (_attn_scores :469-474,
 * di_softmax ops/di_softmax.py:33-61, _attn_context :476-478 with
 * int_gemm_u16i8 backends.py:152-164). Queries t in [0, T) sit at slots
 * S_past + t; slot s is visible iff s <= S_past + t and valid[b][s].
 * out [B][T][n_q*128] int64 = exact sum_s p_s v_s over the paged cache;
 * S_past + T <= min(width * 128, 131071). */
int detllm_attn_prefill(const int8_t* q8, const int64_t* tpos, const int8_t* kpool,
                        const int8_t* vpool, const int32_t* table, int width,
                        const uint8_t* valid, int64_t valid_stride, int B, int T, int S_past,
                        int n_q, int n_kv, int64_t* out, hipStream_t s);

/* Decode attention (one query per row) — model.py:347-381 and the fused
 * Triton kernel ops/fused_attn.py:47-142 it replaces. Scans S <= 131071 slots
 * (further bounded by *s_dev when non-null); scratch [B][n_q][ceil16(S)]
 * int32 is required only when n_q/n_kv * ceil16(S) * 4 > 48 KiB.
 * out [B][n_q*128]. *s_dev above S sets bit 4 of *err. */
int detllm_attn_decode(const int8_t* q8, const int64_t* tpos, const int8_t* kpool,
                       const int8_t* vpool, const int32_t* table, int width,
                       const uint8_t* valid, int64_t valid_stride, int B, int S, int n_q, int n_kv,
                       const int64_t* s_dev, int32_t* scratch, int64_t* out, int32_t* err,
                       hipStream_t s);

/* Split-S decode attention — the same integers as detllm_attn_decode, with
 * each row's slots cut into chunks of `chunk` slots, one block per (row, kv
 * head, chunk) (the reference scans a row in one Triton program,
 * ops/fused_attn.py:47-142). Two launches: scores of each chunk to
 * scores [B][n_q][nsplit * chunk] int32 with per-chunk maxima to
 * cmax [B][n_q][nsplit] int32; then, from the true row maximum and the
 * denominator over all the row's slots, each chunk's partial context to
 * out [nsplit][B][n_q * 128] int64. The context is the sum of the nsplit
 * partials (detllm_merge_rowcol sums them). nsplit = ceil(S / chunk); chunk a
 * multiple of 128, at most 4096, with n_q/n_kv * chunk * 4 <= 48 KiB.
 * Other arguments and err as in detllm_attn_decode. */
int detllm_attn_decode_split(const int8_t* q8, const int64_t* tpos, const int8_t* kpool,
                             const int8_t* vpool, const int32_t* table, int width,
                             const uint8_t* valid, int64_t valid_stride, int B, int S, int n_q,
                             int n_kv, const int64_t* s_dev, int chunk, int32_t* scores,
                             int32_t* cmax, int64_t* out, int32_t* err, hipStream_t s);

/* The chunking detllm_attn_decode_split is tuned for at (B, S, n_q, n_kv):
 * about 1024 blocks, chunks of 256 slots or more. Writes *chunk, *nsplit. */
int detllm_attn_split_plan(int B, int S, int n_q, int n_kv, int* chunk, int* nsplit);

/* Per-step bookkeeping of the graph-captured decode (src/detllm/graphed.py:
 * 112-131: the validity flag of the step's slot, the device scalars holding
 * the write slot and the scanned-slot count, the positions), one launch
 * before each replay:
 * valid[b * valid_stride + slot] = 1, *len_idx = slot, *nslots = slot + 1,
 * pos[b] = pos0[b] + step for b < B. */
int detllm_decode_prologue(uint8_t* valid, int64_t valid_stride, int B, int64_t slot,
                           int64_t* len_idx, int64_t* nslots, int64_t* pos, const int64_t* pos0,
                           int64_t step, hipStream_t s);

/* One decode step's attention block with the Q/K/V epilogue fused in (one
 * query token per row; n_q / n_kv <= 2): detllm_qkv_epilogue with T = 1 —
 * model.py:200-216, :303-358 — followed by detllm_attn_decode — model.py:347-381
 * and ops/fused_attn.py:47-142 — in one launch. Arguments as in those two
 * entry points (P [nsplit][B][(n_q + 2 n_kv) * 128]; the step's slot is
 * *slot_base_dev or slot_base; S <= 131071 slots are scanned, bounded by
 * *s_dev when non-null). out [B][n_q * 128] int64. err as in both. */
int detllm_qkv_attn_decode(const int32_t* P, int nsplit, int64_t split_stride, int B, int n_q,
                           int n_kv, const int64_t* xm, const int64_t* xk,
                           const int64_t* positions, const int64_t* q_m, int64_t q_k,
                           const int64_t* k_m, int64_t k_k, const int64_t* v_m, int64_t v_k,
                           const int64_t* q_norm_m, int64_t q_norm_k, const int64_t* k_norm_m,
                           int64_t k_norm_k, const int64_t* qs_m, int64_t qs_k,
                           const int64_t* kq_m, const int64_t* kq_k, const int64_t* ks_m,
                           const int64_t* ks_k, const int64_t* vq_m, const int64_t* vq_k,
                           const int16_t* cos_t, const int16_t* sin_t, int64_t max_pos,
                           int8_t* kpool, int8_t* vpool, const int32_t* table, int width,
                           const int64_t* slot_base_dev, int64_t slot_base,
                           const uint8_t* valid, int64_t valid_stride, int S,
                           const int64_t* s_dev, int32_t* scratch, int64_t* out, int32_t* err,
                           hipStream_t s);

/* detllm_qkv_attn_decode, and the merge statistics of its output for
 * detllm_igemv_merge_ext: om [n_q * 128] the merge's per-column factor
 * os_m * col_m (model.py:404-409); ext [B][n_kv][2] int64: for row b and kv
 * head h, the largest v and the largest ~v over v = out[b][c] * om[c]
 * (int64, wrapping) for the columns c of h's query heads, and 0 — the
 * extremes dyadic.py:133-136 reduces over the row. */
int detllm_qkv_attn_decode_ext(const int32_t* P, int nsplit, int64_t split_stride, int B,
                               int n_q, int n_kv, const int64_t* xm, const int64_t* xk,
                               const int64_t* positions, const int64_t* q_m, int64_t q_k,
                               const int64_t* k_m, int64_t k_k, const int64_t* v_m, int64_t v_k,
                               const int64_t* q_norm_m, int64_t q_norm_k,
                               const int64_t* k_norm_m, int64_t k_norm_k, const int64_t* qs_m,
                               int64_t qs_k, const int64_t* kq_m, const int64_t* kq_k,
                               const int64_t* ks_m, const int64_t* ks_k, const int64_t* vq_m,
                               const int64_t* vq_k, const int16_t* cos_t, const int16_t* sin_t,
                               int64_t max_pos, int8_t* kpool, int8_t* vpool,
                               const int32_t* table, int width, const int64_t* slot_base_dev,
                               int64_t slot_base, const uint8_t* valid, int64_t valid_stride,
                               int S, const int64_t* s_dev, int32_t* scratch, int64_t* out,
                               int32_t* err, const int64_t* om, int64_t* ext, hipStream_t s);

/* ------------------------------------------- operator-level entry points -- */
/* One reference function each (rows = leading dims flattened, C = last dim). */

/* dyadic.quant_i8_pertoken — src/detllm/dyadic.py:93-105 */
int detllm_op_quant_i8_pertoken(const int64_t* x, const int64_t* m, const int64_t* k, int R,
                                int C, int8_t* x8, int64_t* mo, int64_t* ko, hipStream_t s);

/* dyadic.requant_i32_common — dyadic.py:108-120 (col_m [G][C], row r uses
 * group r % G) */
int detllm_op_requant_i32_common(const int64_t* P, const int64_t* row_k, const int64_t* col_m,
                                 int G, int64_t col_k, int tb, int R, int C, int32_t* y,
                                 int64_t* ko, hipStream_t s);

/* dyadic.requant_i8_rowcol — dyadic.py:123-139 */
int detllm_op_requant_i8_rowcol(const int64_t* P, const int64_t* row_m, const int64_t* row_k,
                                const int64_t* col_m, int64_t col_k, int R, int C, int8_t* y8,
                                int64_t* mo, int64_t* ko, hipStream_t s);

/* dyadic.requant_i8_static — dyadic.py:142-163 (operands materialised per
 * element) */
int detllm_op_requant_i8_static(const int64_t* P, const int64_t* row_m, const int64_t* row_k,
                                const int64_t* col_m, const int64_t* col_k, const int64_t* s_m,
                                const int64_t* s_k, int64_t n, int8_t* y8, hipStream_t s);

/* dyadic.residual_renorm (mode 0) / residual_add (mode 1) — dyadic.py:174-206 */
int detllm_op_residual(int mode, const int64_t* h, const int64_t* k_res, const int64_t* d,
                       const int64_t* dm, const int64_t* dk, int R, int C, int32_t* h_out,
                       int64_t* k_out, hipStream_t s);

/* ops.di_rmsnorm (gamma_m null, int32 out) / di_rmsnorm_gamma (int64 out) —
 * src/detllm/ops/di_rmsnorm.py:33-64 */
int detllm_op_rmsnorm(const int64_t* x, const int64_t* gamma_m, int R, int C, int32_t* y32,
                      int64_t* y64, hipStream_t s);

/* ops.di_softmax — src/detllm/ops/di_softmax.py:33-61 */
int detllm_op_softmax(const int64_t* x, const int64_t* m, const int64_t* k, const uint8_t* valid,
                      int has_clip, int64_t clip_c, int p_out_bits, int R, int C, int32_t* probs,
                      hipStream_t s);

/* ops.di_exp — src/detllm/ops/di_exp.py:21-37 */
int detllm_op_di_exp(const int64_t* x, const int64_t* m, const int64_t* k, int R, int C,
                     int64_t* res, int64_t* tpos, hipStream_t s);

/* ops.di_swiglu — src/detllm/ops/di_swiglu.py:39-58 */
int detllm_op_swiglu(const int64_t* gate, const int64_t* gm, const int64_t* gk,
                     const int64_t* up, const int64_t* um, const int64_t* uk, int R, int C,
                     int64_t* y, int64_t* ym, int64_t* yk, hipStream_t s);

/* ops.apply_int_rope — src/detllm/ops/rope.py:38-55 (head_dim 128); a
 * position outside [-max_pos, max_pos) sets bit 2 of *err */
int detllm_op_rope(const int64_t* x, const int64_t* pos, const int16_t* cos_t,
                   const int16_t* sin_t, int64_t max_pos, int64_t rows, int64_t* y,
                   int32_t* err, hipStream_t s);

/* Elementwise primitives: op 0 isqrt (intmath.py:180-202, int_prims.py:31-44),
 * 1 ilog2_floor (intmath.py:164-177, int_prims.py:47-55), 2 norm_scale
 * (dyadic.py:75-90), 3 fit_dyadic_ratio (dyadic.py:52-72), 4
 * scaled_round_div (dyadic.py:45-49); and the device forms the fused kernels
 * use for the same functions: 5 fit_dyadic_ratio(a, 127) (constant-divisor
 * path), 6 isqrt by the wave-parallel search, 7 the SwiGLU sigmoid division
 * round_half_away_div(a << 7, b) (ops/di_swiglu.py:52-55) in the fused
 * kernels' single-precision form, for 0 <= a <= b < 2^24; and the fp64
 * estimate forms, each valid under the bound intops.h states for it:
 * 8 rhad(a c, b) for a >= 0 (rhad_est), 9 its signed form (rhad_est_signed),
 * 10 clamp_i8(rhad(a, b)) (rhad_est_i8), 11 sign(a) rhad(|a| c, b) with the
 * remainder step (rhad_est_corr_signed), 12 DI-Exp of -a with tpos b
 * (dexp_est, ops/di_exp.py:27-37), 13 the same from a = t - n with t = b
 * (dexp_est_sp), 14 the DI-Exp constant of (m, k) = (a, b) (di_exp_tpos_fast,
 * model.py:355-358), 15 isqrt(a) (isqrt_est). */
int detllm_op_scalar(int op, const int64_t* a, const int64_t* b, const int64_t* c, int64_t n,
                     int64_t* o1, int64_t* o2, hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif /* DETLLM_HIP_H */
