// bonsai_p40.h -- C ABI of the MI355X (gfx950) PQ2_0 matmul path.
//
// Drop-in for the reference header include/bonsai_p40.h of
// boetti-dev/p40-kernel: every declaration of that header is kept with the
// same name, argument order, argument meaning and return-code convention, so
// C++ host code written against it links against libbonsai_p40.so unchanged.
// Where the reference's host and device code disagree, the reference name
// keeps what the reference LIBRARY does when it reads memory (the FWHT's
// 1024-entry signs), and its rounding follows the host code (below).
// The library is written for AMD CDNA4 (gfx950) in HIP; `bonsai_stream` is a
// hipStream_t (NULL = the default stream).
//
// Conventions shared by every entry point (reference: gemv_p40.cu:200-219,
// gemm_p40.cu:143-154, gemv_repack_p40.cu:196-220, elementwise_p40.cu:75-80):
//   * all pointers are device pointers owned by the caller; nothing is
//     allocated and nothing synchronises -- work is enqueued on `stream`;
//   * return 1 for invalid arguments, 0 for an empty no-op, otherwise the
//     hipError_t of the launch (so 0 = enqueued).  Callers test `!= 0`;
//   * a NULL device pointer that the requested work would read or write is an
//     invalid argument (1, nothing launched), where the reference launches
//     anyway; optional pointers (signs, norm weights, status) may be NULL.
//     The empty no-ops (n_out <= 0, n_tok <= 0, ...) still return 0 first, as
//     in the reference;
//   * block_pq2_0 = 34 bytes (fp16 d, 32 bytes of 2-bit codes, element j in
//     byte j/4 at bits 2(j%4), value (code-1)*d); block_q8_1 = 36 bytes (fp16
//     d, int16 sum s stored as raw bits, 32 int8 in the PQ2_0-native permuted
//     order: position j holds element 16(j>>4) + 4(j&3) + ((j>>2)&3));
//   * Q8_1 buffers must be 4-byte aligned.  PQ2_0 weights need only the
//     2-byte alignment of the format; 16-byte aligned weights with
//     n_in % 1024 == 0 take the streaming fast path.
//   * rounding follows the reference HOST code (src/pq2_0.h:99-126,
//     src/p40_common.h:82-114): q = lroundf(x/d) (ties away from zero) and the
//     fp16 scale rounds ties away from zero, so Q8_1 bytes equal the host's.
#pragma once

#include <cstdint>
#include <cstddef>

#ifdef __cplusplus
extern "C" {
#endif

// Opaque stream handle (a hipStream_t), reference include/bonsai_p40.h:16.
typedef void * bonsai_stream;

// --- decode (batch = 1) matrix-vector -------------------------------------
// y[n_out] = W[n_out, n_in] . x with x already in permuted Q8_1 (xq).
// Replaces include/bonsai_p40.h:21-22 (src/kernels/gemv_p40.cu:210-219).
// Errors: 1 if n_in <= 0 or n_in % 128 != 0 or xq is not 4-byte aligned;
// 0 (no-op) if n_out <= 0; then 1 if n_out >= 2^30 or n_in / 128 > 2^24.
int bonsai_p40_gemv(const void * W, const void * xq, float * y,
                    int64_t n_out, int64_t n_in, bonsai_stream stream);

// Quantise n floats to permuted Q8_1 (n/32 blocks of 36 bytes).
// Replaces include/bonsai_p40.h:25 (src/kernels/gemv_p40.cu:200-208).
// Errors: 1 if n <= 0 or n % 32 != 0.
int bonsai_p40_quant_activations(const float * x, void * out, int64_t n, bonsai_stream stream);

// --- prefill (batch > 1) ----------------------------------------------------
// Y[n_out, n_tok] (row-major, Y[r*n_tok + t]) = W . X, X in permuted Q8_1,
// chunk-major: block (c, t) at index c*n_tok + t (src/kernels/gemm_p40.cu:75).
// Replaces include/bonsai_p40.h:29-30 (src/kernels/gemm_p40.cu:143-154).
// n_tok == 1 runs the decode GEMV; 2 tokens the streaming kernel with
// per-token activation planes; 3..8 the block-diagonal 16x16x64 int8 MFMA
// kernel, except 4 tokens on 1024-, 5120- and 6144-column rows and 3 on
// 1024- and 6144-column rows, which take the 4x4x4 int8 MFMA streaming
// kernel; 9..16 the streamed 16x16x32 int8 MFMA kernel; larger n_tok the
// f16-MFMA tile GEMM (other alignments: 64-bit-offset MFMA kernels).  The
// GEMV and the streamed small-batch kernels subtract each Q8_1 block's
// stored sum s as the reference does (src/pq2_0.h:169); the tile GEMMs and
// the kernels for other alignments multiply (code - 1) by q directly and do
// not read s.  The two agree for blocks whose s is the sum of their q, which
// holds for every block this library's or the reference's quantiser writes.  Errors: 1 if n_in <= 0 or n_in % 128 != 0, Xq is not 4-byte or W
// not 2-byte aligned, or n_out, n_tok or n_in / 128 is too large for the
// launch; 0 (no-op) if n_out <= 0 or n_tok <= 0.
int bonsai_p40_gemm(const void * W, const void * Xq, float * Y,
                    int64_t n_out, int64_t n_in, int64_t n_tok, bonsai_stream stream);

// bonsai_p40_gemm with a caller workspace (an addition; the reference has no
// counterpart): where the long-prompt kernel runs (the rows bonsai_p40_gemm
// gives its 256- or 160-row tiles) on a matrix of 8192 rows or more, Xq is
// first converted once into the workspace (each q byte as f16, each d as
// fp32: both exact), and the tiles take the activation from there by DMA
// instead of converting it per tile; elsewhere it runs bonsai_p40_gemm.
// Y is bit-identical to bonsai_p40_gemm's.  workspace: 16-byte aligned,
// bonsai_p40_gemm_workspace_bytes(n_in, n_tok) bytes; NULL (any ws_bytes)
// runs bonsai_p40_gemm.  The workspace is scratch for the call (stream-
// ordered: calls that share one must be ordered on one stream).  Errors: those
// of bonsai_p40_gemm, and 1 if workspace is not 16-byte aligned or ws_bytes is
// smaller than the size the call needs.
int bonsai_p40_gemm_ws(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_in,
                       int64_t n_tok, void * workspace, int64_t ws_bytes, bonsai_stream stream);
// Workspace bytes bonsai_p40_gemm_ws needs (n_tok * n_in / 32 * 68); 0 where
// it needs none (n_in or n_tok <= 0, or the converted activation would not
// be addressable with 32-bit offsets: 2 GiB and more, the call then runs
// bonsai_p40_gemm whatever the workspace).
int64_t bonsai_p40_gemm_workspace_bytes(int64_t n_in, int64_t n_tok);

// --- aligned repacked layout ------------------------------------------------
// Size-neutral row: d[nb] fp16, then 4 planes of nb 8-byte code units; unit
// u = plane*nb + block at byte 2*nb + 8u (src/pq2_0_repack.h:46-57).
// src and dst must not overlap.  Errors: 1 if n_in % 128 != 0, n_out <= 0 or
// n_in/128 is not a positive multiple of 8.
// Replaces include/bonsai_p40.h:35 (src/kernels/gemv_repack_p40.cu:196-207).
int bonsai_p40_repack(const void * src, void * dst, int64_t n_out, int64_t n_in, bonsai_stream stream);
// y = W_repacked . x for fp32 x (quantised to Q8_1 inside the kernel).
// Replaces include/bonsai_p40.h:36-37 (src/kernels/gemv_repack_p40.cu:209-220).
// Errors: as bonsai_p40_repack, plus 1 if W is not 8-byte aligned (its 8-byte
// code units are read whole) or, on widths without the streaming kernel, the
// quantised activation (n_in/32 * 40 bytes) does not fit the 160 KiB LDS of a
// workgroup.
int bonsai_p40_gemv_repack(const void * W, const float * x, float * y,
                           int64_t n_out, int64_t n_in, bonsai_stream stream);

// --- transforms -----------------------------------------------------------------
// In-place normalised Sylvester-Hadamard transform in blocks of 1024.  signs
// (optional, NULL = all +1) has 1024 entries, used by EVERY block: the meaning
// of the reference device kernel (elementwise_p40.cu:17-41, signs[i] with
// i < 1024), so a buffer sized for the reference library is never read past.
// Stage order h = 1..512 as the host, so the result is bit-identical to the
// host fwht_blocks() given that vector tiled to length n.  Errors: 1 if
// n <= 0 or n % 1024 != 0.  Replaces include/bonsai_p40.h:41
// (elementwise_p40.cu:75-80).
int bonsai_p40_fwht(float * x, const float * signs, int64_t n, bonsai_stream stream);

// Not on the PQ2_0 matmul path; kept so the reference's symbol set links.
// rmsnorm: y = x * (1/sqrt(mean(x^2) + eps)) * w per row (src/ops.h:13-22).
int bonsai_p40_rmsnorm(const float * x, const float * w, float * y,
                       int64_t n_rows, int64_t n, float eps, bonsai_stream stream);
// gdn_step / attn are outside this library's scope: they return 2
// ("not implemented") without touching memory.
int bonsai_p40_gdn_step(float * state, const float * q, const float * k, const float * v,
                        const float * g, const float * beta, float * out,
                        int n_k_heads, int n_v_heads, int K, int V, bonsai_stream stream);
int bonsai_p40_attn(const float * q, const float * k, const float * v, float * out,
                    int n_tok, int n_head, int n_head_kv, int head_dim, float scale,
                    bonsai_stream stream);

// --- additions (no counterpart in the reference header) -------------------------
// Every addition that takes `signs` reads a length-n vector (block b uses
// signs[1024 b ..]), the host form of src/fwht.h:38-42.

// bonsai_p40_fwht with the host's length-n signs (block b uses
// signs[1024 b .. 1024 b + 1023]): bit-identical to fwht_blocks(x, signs, n).
// Errors as bonsai_p40_fwht.
int bonsai_p40_fwht_signs_n(float * x, const float * signs, int64_t n, bonsai_stream stream);

// Fused decode pre-pass: xq = Q8_1(FWHT(signs .* x)) for one token of n floats
// (x is not modified).  One launch in place of bonsai_p40_fwht followed by
// bonsai_p40_quant_activations (elementwise_p40.cu:17-41 + gemv_p40.cu:168-196),
// bit-identical to the host fwht_blocks + quantize_row_q8_1(permute = true).
// Errors: 1 if n <= 0 or n % 1024 != 0.
int bonsai_p40_fwht_quant(const float * x, const float * signs, void * xq, int64_t n,
                          bonsai_stream stream);

// Batched pre-pass for the GEMM: X is [n_tok][n] fp32 (token rows); each token
// is optionally rotated (rotate != 0: FWHT with signs, n % 1024 == 0) and
// quantised on its own, written chunk-major (block (c, t) at c*n_tok + t) --
// the Xq layout bonsai_p40_gemm consumes, which the reference API has no
// producer for.  Errors: 1 if n <= 0, n % 32 != 0 (n % 1024 with rotate),
// n_tok <= 0 or n_tok > 65535 (one grid row per token), n * n_tok > 2^40, X or
// Xq is NULL, Xq is not 4-byte aligned, or signs is given without rotate.
int bonsai_p40_quant_tokens(const float * X, const float * signs, void * Xq, int64_t n,
                            int64_t n_tok, int rotate, bonsai_stream stream);

// Layer-input pre-pass: Xq = Q8_1(FWHT(signs .* RMSNorm(x, w, eps))) for n_tok
// token rows of n floats, one launch in place of bonsai_p40_rmsnorm followed by
// bonsai_p40_fwht and bonsai_p40_quant_activations (elementwise_p40.cu:17-41,
// 48-88 + gemv_p40.cu:168-196; RMSNorm as src/ops.h:13-22).  The sum of squares
// is accumulated in fp64 in one order shared by every normalising entry point
// (whatever n_tok), so the scale can differ from the reference's sequential
// fp32 sum by that sum's rounding; the rest is bit-identical to the
// host FWHT and quantiser.  Output chunk-major (block (c, t) at c*n_tok + t: the
// GEMM's Xq; for n_tok == 1 the GEMV's xq).  x, w and signs are [n_tok][n], [n]
// and [n] (signs may be NULL).  Errors: 1 if n <= 0, n % 1024 != 0, x or w is
// NULL, or xq is not 4-byte aligned; 0 (no-op) if n_tok <= 0.
int bonsai_p40_rmsnorm_fwht_quant(const float * x, const float * w, const float * signs, void * xq,
                                  int64_t n, int64_t n_tok, float eps, bonsai_stream stream);

// FFN glue of the decode chain: xq = Q8_1(FWHT(signs .* (silu(gate) * up)))
// with silu(g) = g / (1 + exp(-g)) (src/ops.h:27-31), one launch.
// Errors: 1 if n <= 0 or n % 1024 != 0.
int bonsai_p40_swiglu_fwht_quant(const float * gate, const float * up, const float * signs,
                                 void * xq, int64_t n, bonsai_stream stream);

// Fused decode GEMV from the fp32 activation: y = W . Q8_1(FWHT(signs .* x)),
// one launch in place of bonsai_p40_fwht_quant followed by bonsai_p40_gemv
// (the reference runs them as two kernels: elementwise_p40.cu:75-80 +
// gemv_p40.cu:200-219).  Every workgroup rotates and quantises x into its own
// LDS with the pre-pass's device code, so the Q8_1 bytes are the host's; on
// the model widths (n_in/128 in {8, 40, 48, 80, 96, 136}) with 16-byte
// aligned W, x and signs, y is bit-identical to the two-call sequence.  x is
// not modified; signs may be NULL.  Errors: 1 if n_in <= 0, n_in % 1024 != 0,
// x is NULL, or (other widths) the Q8_1 activation, 36 bytes per 32 columns,
// does not fit in a workgroup's LDS less 1 KiB (n_in > 144384 with MI355X's
// 160 KiB); 0 (no-op) if n_out <= 0.
int bonsai_p40_fwht_gemv(const void * W, const float * x, const float * signs, float * y,
                         int64_t n_out, int64_t n_in, bonsai_stream stream);

// Decode GEMV from an fp32 activation that is already in the weights' basis:
// y = W . Q8_1(x), one launch in place of bonsai_p40_quant_activations
// followed by bonsai_p40_gemv -- the reference's ggml hook sequence
// (integrations/prismml/bonsai-p40.diff:283-291), which needs a Q8_1 scratch
// buffer; this needs none.  Every workgroup quantises x into its own LDS with
// the quantiser's device code (host rounding); on the model widths with
// 16-byte aligned W and x, y is bit-identical to the two-call sequence.
// Errors: 1 if n_in <= 0, n_in % 1024 != 0, x is NULL, or (other widths) the
// Q8_1 activation does not fit in a workgroup's LDS less 1 KiB (n_in > 144384
// with MI355X's 160 KiB); 0 (no-op) if n_out <= 0.
int bonsai_p40_quant_gemv(const void * W, const float * x, float * y, int64_t n_out, int64_t n_in,
                          bonsai_stream stream);

// Grouped decode GEMV: y[m] = W[m] . xq for the n_mat (1..4) matrices that
// multiply one activation (q, k and v; gate and up), in one launch over the
// concatenated rows (the reference launches one GEMV per matrix,
// gemv_p40.cu:210-219).  W, y and n_out are host arrays of n_mat entries;
// every W[m] has n_in columns.  y[m] is bit-identical to bonsai_p40_gemv on
// W[m] alone.  Errors: as bonsai_p40_gemv, plus 1 if n_mat is outside 1..4,
// an array is NULL or a matrix has more than 2^30 - 1 rows; matrices with
// n_out[m] <= 0 are skipped (0 if all are).
int bonsai_p40_gemv_group(const void * const * W, float * const * y, const int64_t * n_out, int n_mat,
                          const void * xq, int64_t n_in, bonsai_stream stream);

// Grouped form of bonsai_p40_fwht_gemv: y[m] = W[m] . Q8_1(FWHT(signs .* x)),
// one rotation per workgroup for the whole group; y[m] is bit-identical to
// bonsai_p40_fwht_gemv on W[m] alone.  Errors: as bonsai_p40_fwht_gemv and
// bonsai_p40_gemv_group.
int bonsai_p40_fwht_gemv_group(const void * const * W, float * const * y, const int64_t * n_out, int n_mat,
                               const float * x, const float * signs, int64_t n_in, bonsai_stream stream);

// Layer-input grouped decode GEMV: y[m] = W[m] . Q8_1(FWHT(signs .* RMSNorm(x,
// norm_w, eps))) for the n_mat (1..4) matrices that read one normalised layer
// input (q/k/v after the attention norm, gate/up after the FFN norm), in one
// launch in place of bonsai_p40_rmsnorm + bonsai_p40_fwht +
// bonsai_p40_quant_activations + one bonsai_p40_gemv per matrix
// (elementwise_p40.cu:48-88, 17-41 + gemv_p40.cu:168-219).  Every workgroup
// normalises, rotates and quantises x into its own LDS; the sum of squares is
// fp64, added in the one order every normalising entry point uses, so y[m]
// equals bonsai_p40_rmsnorm_fwht_quant followed by bonsai_p40_gemv_group.  x and norm_w have n_in floats; signs may be NULL.
// Errors: as bonsai_p40_fwht_gemv_group, plus 1 if norm_w is NULL.
int bonsai_p40_rmsnorm_fwht_gemv_group(const void * const * W, float * const * y, const int64_t * n_out,
                                       int n_mat, const float * x, const float * norm_w, const float * signs,
                                       int64_t n_in, float eps, bonsai_stream stream);

// FFN gate/up with its SwiGLU glue in one launch (src/ops.h:27-31 after the
// gate and up GEMVs):  hq = Q8_1(FWHT(h_signs .* silu(Wg . a) * (Wu . a)))
// with a = Q8_1(FWHT(x_signs .* RMSNorm(x, norm_w, eps))) (norm_w NULL: no
// RMSNorm).  In place of bonsai_p40_rmsnorm_fwht_gemv_group on {Wg, Wu}
// followed by bonsai_p40_swiglu_fwht_quant (the reference runs rmsnorm, fwht,
// quant_activations, two gemv and the glue as separate kernels); hq is the
// same bytes, ready for the down projection's bonsai_p40_gemv.  Wg and Wu are
// n_ff x n_embd PQ2_0; x, norm_w, x_signs have n_embd floats, h_signs n_ff
// (signs may be NULL); hq has n_ff/32 Q8_1 blocks.
// workspace: BONSAI_P40_FFN_WORKSPACE_BYTES(n_ff) device bytes, 16-byte
// aligned, ZERO-FILLED before its first use.  Its first
// BONSAI_P40_FFN_SYNC_BYTES are flags, then 2 n_ff words through which the
// gate and up rows pass from the workgroups that compute them to the one that
// finishes their 1024-block; a completed call leaves all of it zero again
// (do not modify it between calls).  Calls that may run at the same time
// need their own workspaces.  status (device, may be NULL): the kernel adds 1
// for each internal wait that gave up (it then leaves hq partly unwritten and
// the workspace must be zero-filled again).  On widths without the one-launch
// kernel the call runs the grouped GEMV and the glue as two launches and the
// rows stay in the workspace as plain fp32.  Errors: 1 if a pointer is NULL
// or misaligned, n_ff or n_embd <= 0 or not a multiple of 1024.
#define BONSAI_P40_FFN_SYNC_BYTES 256
#define BONSAI_P40_FFN_WORKSPACE_BYTES(n_ff) (BONSAI_P40_FFN_SYNC_BYTES + 8 * (int64_t)(n_ff))
int bonsai_p40_ffn_gate_up_swiglu(const void * Wg, const void * Wu, const float * x, const float * norm_w,
                                  const float * x_signs, const float * h_signs, void * hq, int64_t n_ff,
                                  int64_t n_embd, float eps, void * workspace, uint32_t * status,
                                  bonsai_stream stream);

// bonsai_p40_ffn_gate_up_swiglu without a workspace argument, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid allocation).  No counterpart in the
// reference.  The workspace is a static device array inside the library of
// BONSAI_P40_FFN_WORKSPACE_BYTES(BONSAI_P40_FFN_NOALLOC_MAX_NFF) bytes (~512
// KiB), one per GPU for the life of the process; the call allocates nothing
// (two kernel launches: a check that repairs the array after a wait that gave
// up, then the fused launch).  Every call
// on one GPU shares that array, so calls that overlap on one GPU (different
// streams, different host threads) race and must not be issued.  Errors: as
// bonsai_p40_ffn_gate_up_swiglu, plus 1 if n_ff > BONSAI_P40_FFN_NOALLOC_MAX_NFF;
// the hipError_t of the one-time symbol lookup if it fails.
#define BONSAI_P40_FFN_NOALLOC_MAX_NFF 65536
int bonsai_p40_ffn_gate_up_swiglu_noalloc(const void * Wg, const void * Wu, const float * x,
                                          const float * norm_w, const float * x_signs, const float * h_signs,
                                          void * hq, int64_t n_ff, int64_t n_embd, float eps, uint32_t * status,
                                          bonsai_stream stream);

// Reference ternary weight quantiser: n fp32 weights (n % 128 == 0, rows of a
// matrix back to back) -> n/128 block_pq2_0 with d = amax rounded to fp16
// half away from zero and code = clamp(lroundf(x / amax) + 1, 0, 3); bytes
// equal quantize_row_pq2_0 (src/pq2_0.h:74-90) for finite inputs.  A
// load-time transform; the reference has it only on the host.  Errors: 1 if
// n <= 0, n % 128 != 0, a pointer is NULL, x is not 4-byte or w not 2-byte
// aligned.
int bonsai_p40_quantize_pq2_0(const float * x, void * w, int64_t n, bonsai_stream stream);
// Its inverse: y = (code - 1) * d for n weights (src/pq2_0.h:62-71), exact.
// Errors as bonsai_p40_quantize_pq2_0.
int bonsai_p40_dequantize_pq2_0(const void * w, float * y, int64_t n, bonsai_stream stream);

// ---------------------------------------------------------------------------
// Decode chain: a sequence of dependent decode steps run by ONE persistent
// launch (no counterpart in the reference, whose host launches every matmul
// and glue op separately; each step computes exactly what the entry point
// named beside its kind computes).  One workgroup per CU; between two steps
// every workgroup waits at a grid-wide barrier (flag words in the workspace,
// bounded polling), and while it waits its waves already stream the first
// weight units of the next GEMV step into LDS.  A step's input may be an
// earlier step's output.
//   BONSAI_P40_CHAIN_Q8:     y[m] = W[m] . x, x the permuted Q8_1 of n_in
//                            values (bonsai_p40_gemv_group);
//   BONSAI_P40_CHAIN_FWHT:   x fp32: bonsai_p40_fwht_gemv_group (signs NULL or
//                            length n_in);
//   BONSAI_P40_CHAIN_RMSNORM_FWHT: x fp32: bonsai_p40_rmsnorm_fwht_gemv_group
//                            with norm_w and eps;
//   BONSAI_P40_CHAIN_SWIGLU: no matrix: q_out = Q8_1(FWHT(signs .* swiglu(x,
//                            x2))) over n_in values (bonsai_p40_swiglu_fwht_quant).
// Widths: FWHT / RMSNORM_FWHT n_in in {5120, 6144}; Q8 n_in in {5120, 6144,
// 17408}; SWIGLU n_in % 1024 == 0.  Up to 4 matrices per step (16-byte
// aligned, < 2 GiB each); x, x2, norm_w and signs 16-byte aligned, x of Q8
// steps and q_out 4-byte aligned.
#define BONSAI_P40_CHAIN_Q8 0
#define BONSAI_P40_CHAIN_FWHT 1
#define BONSAI_P40_CHAIN_RMSNORM_FWHT 2
#define BONSAI_P40_CHAIN_SWIGLU 3
typedef struct bonsai_p40_chain_step {
    int kind;
    int n_mat;                  // 1..4 (0 for SWIGLU)
    const void * W[4];
    float * y[4];
    int64_t n_out[4];
    int64_t n_in;
    const void * x;             // input (Q8_1 bytes or fp32; SWIGLU: gate rows)
    const float * x2;           // SWIGLU: up rows
    const float * norm_w;       // RMSNORM_FWHT: n_in weights
    const float * signs;        // NULL or n_in values of +-1
    void * q_out;               // SWIGLU: Q8_1 output (n_in/32 blocks)
    float eps;                  // RMSNORM_FWHT
} bonsai_p40_chain_step;
// Bytes of device memory a plan of n_steps steps needs.
int64_t bonsai_p40_chain_plan_bytes(int n_steps);
// Checks every step and writes the device form of the chain into plan (device
// memory of bonsai_p40_chain_plan_bytes bytes) with a blocking copy: a set-up
// call, made once per chain and device, before any launch that uses the plan
// (and outside stream capture).  Errors: 1 if a step is invalid (nothing is
// written), else the copy's hipError_t.
int bonsai_p40_chain_plan(const bonsai_p40_chain_step * steps, int n_steps, void * plan);
// Workspace of bonsai_p40_chain_run: one flag word per workgroup and, in its
// last word, the abort word.  Zero-fill it once before its first use and
// then leave it alone: every completed launch leaves it ready for the next.
// Launches that may run at the same time need their own workspaces.
#define BONSAI_P40_CHAIN_WORKSPACE_BYTES 4096
// Runs a planned chain on the device it was planned on.  status (device, may
// be NULL): incremented for every barrier wait that gave up (the chain's
// workgroups could not all be resident, e.g. beside another kernel); the
// first give-up sets the workspace's abort word, on which every workgroup
// leaves at its next barrier or poll, so a failed launch ends within about
// one wait bound.  The outputs of such a launch are not valid and the
// workspace must be zero-filled again: a launch that finds the abort word
// set adds 1 to status and does nothing.  Errors: 1 on bad arguments, else
// the launch's hipError_t.
int bonsai_p40_chain_run(const void * plan, int n_steps, void * workspace, uint32_t * status,
                         bonsai_stream stream);

// Test hook: out[r * (n_in/32) + c] = the int32 chunk dot sum_k (code-1)*q of
// row r, chunk c, computed by the same device code path as bonsai_p40_gemv
// (the value of src/pq2_0.h:149-177 before scaling).  Errors as bonsai_p40_gemv.
int bonsai_p40_chunk_dots(const void * W, const void * xq, int32_t * out,
                          int64_t n_out, int64_t n_in, bonsai_stream stream);

// Tuning hook: the library reads its BONSAI_* environment variables (kernel
// variant selectors used by tests and sweeps) once per process, at the first
// call that needs one; this re-reads them after a caller changed them.
// Thread-safe; launches already enqueued keep the variants they were given.
// Returns 0.
int bonsai_p40_reload_tuning(void);

// Measurement helper: a streaming read of `bytes` (16-byte aligned, multiple
// of 16) with `blocks` workgroups of 256 lanes -- the achievable-HBM-bandwidth
// ceiling the GEMV is compared with (the role of the reference's
// tools/bwtest.cu).  `out` needs `blocks` words; it is written only in a
// practically impossible case.  Errors: 1 on bad sizes or alignment.
int bonsai_p40_stream_read(const void * buf, int64_t bytes, uint32_t * out, int blocks,
                           bonsai_stream stream);

// Measurement helper: MFMA peak probe.  `blocks` workgroups of 4 waves, each
// wave issuing iters * 4 independent back-to-back MFMAs of one kind (0 = int8
// v_mfma_i32_16x16x64_i8, 32768 ops each; 1 = f16 v_mfma_f32_16x16x32_f16,
// 16384 ops each).  clk (2 * blocks words) receives, per workgroup, the
// shader-clock and real-time (hipDeviceAttributeWallClockRate) deltas of its
// first wave's loop, from which the clock the MFMAs ran at follows.  sink
// needs `blocks` words.  Errors: 1 on bad arguments.
int bonsai_p40_mfma_probe(int kind, int blocks, int iters, uint64_t * clk, uint32_t * sink,
                          bonsai_stream stream);

// Measurement helper: does the VALU work while the matrix core does?
// `blocks` workgroups of 4 waves; per iteration each wave issues 4 independent
// v_mfma_f32_16x16x32_f16 (mode 0 or 2) and nf x 16 independent fp32 FMAs
// (mode 1 or 2).  Time modes 0, 1 and 2 with events: mode 2 near the larger
// of the other two means overlap, near their sum means the two pipes take
// turns.  Mode 3 is the prefill GEMM's chunk step alone (4 MFMAs with a zero
// accumulator input, then 16 FMAs folding their results into accumulators;
// nf unused): the floor of the GEMM's per-chunk cost without operand staging,
// LDS reads and barriers.  sink needs `blocks` words.  Errors: 1 on bad
// arguments.
int bonsai_p40_overlap_probe(int mode, int nf, int blocks, int iters, uint32_t * sink, bonsai_stream stream);

// Measurement helper: the decode GEMV's weight stream alone -- the unit
// LDS-DMA schedule bonsai_p40_gemv runs for an n_out x n_in PQ2_0 matrix
// (n_in 5120 or 17408; same units, grid, wave numbering, ring depth, issue
// rounds and waits), with no activation and no arithmetic: the floor the
// GEMV's own addressing puts under it (the role of the reference's
// tools/bwtest.cu:70-90).  W 4-byte aligned, under 2 GiB; sink needs one word
// per CU and is written only in a practically impossible case.  Errors: 1 on
// other widths, bad sizes or alignment.
int bonsai_p40_unit_dma_probe(const void * W, int64_t n_out, int64_t n_in, uint32_t * sink,
                              bonsai_stream stream);

// Measurement: one empty kernel (`blocks` workgroups of `threads` threads,
// 1..1024); replayed back to back it gives the cost of a launch that waits for
// the one before it -- the floor under every kernel of a decode chain.
// Errors: 1 on bad arguments.
int bonsai_p40_launch_probe(int blocks, int threads, uint32_t * sink, bonsai_stream stream);

#ifdef __cplusplus
}
#endif
