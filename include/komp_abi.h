/* C ABI of the MI355X (gfx950) decode path of COMP: activation quantizers, the Q4_0 / TQ2_0 decode GEMVs of the
 * reference, batched matrix-core GEMMs, weight splitting on the device, and the ggml formats Q8_0, IQ4_NL and Q4_K
 * (declared further below) through the same entries.
 *
 * Plain C: pointers are device pointers (HIP), sizes are int64_t, `stream` is a hipStream_t passed as void*
 * (NULL = the default stream).  Every call is asynchronous on `stream` and allocates nothing.  Each entry validates
 * shapes, strides and alignment first and returns a nonzero status without touching the GPU when they are wrong;
 * komp_last_error() then describes the problem.  Nothing aborts.  The library keeps no state between calls except
 * the optional dispatch timing and wave stamps of the tuning harness (komp_timing_*, komp_stamps_*).
 *
 * Layouts are the reference's split planes (src/komp/kernels.py:3-7, src/komp/host.py:16-31):
 *   Q4_0 weights   WQ uint8 [N][SW] (row r at WQ + r*SW; 16 quant bytes per block of 32, ggml order),
 *                  WS int16 [N][K/32] (f16 bit patterns, dense)
 *   TQ2_0 weights  WQ uint8 [N][SW] (64 quant bytes per block of 256), WS int16 [N][K/256]
 *   q8_0 acts      XQ int8 [M][K], XD f32 [M][K/32] (holding f32(f16(d)))
 *   q8_K acts      XQ int8 [M][K], XD f32 [M][K/256], XB int16 [M][K/16] bsums (optional)
 *   outputs        Y f32 [M][N]; S int32 [M][N][K/block] exact block dots (optional, verification)
 */
#ifndef KOMP_ABI_H
#define KOMP_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KOMP_ABI_VERSION 1

/* status codes */
#define KOMP_OK 0
#define KOMP_EINVAL 1 /* bad argument: shape, stride, alignment, knob or mode */
#define KOMP_EHIP 2   /* the HIP runtime reported an error (launch or event) */

/* GEMV modes (src/komp/host.py:13, src/komp/kernels.py:9-11) */
#define KOMP_MODE_BYTES 0     /* every value unpacked to int32 first */
#define KOMP_MODE_DP4A_EMU 1  /* packed-word dot products emulated with shifts and multiplies */
#define KOMP_MODE_DP4A 2      /* packed-word dot products on v_dot4c_i32_i8 */

/* Version of this ABI (KOMP_ABI_VERSION).  No reference counterpart. */
int komp_abi_version(void);

/* Message for the last nonzero status returned on the calling thread ("" if none). */
const char* komp_last_error(void);

/* f32 X [M][K] -> q8_0 planes XQ, XD.  K % 32 == 0; X 16-byte aligned, XQ 4-byte aligned.  `bb` (blocks per
 * program in the reference) must be >= 1; every bb gives the same launch and the same bytes.
 * Replaces: host.quantize q8_0 branch (src/komp/host.py:63-69) launching kernels.quant_q8_0 (src/komp/kernels.py:22-33). */
int komp_quant_q8_0(const float* X, int8_t* XQ, float* XD, int64_t M, int64_t K, int bb, void* stream);

/* f32 X [M][K] -> q8_K planes XQ, XD and, when XB is not NULL, the bsums XB [M][K/16].  K % 256 == 0; X and XQ
 * 16-byte aligned.
 * Replaces: host.quantize q8_K branch (src/komp/host.py:70-72) launching kernels.quant_q8_K (src/komp/kernels.py:36-45);
 * the bsums, which the reference computes on the host (src/komp/host.py:50), come from the kernel. */
int komp_quant_q8_K(const float* X, int8_t* XQ, float* XD, int16_t* XB, int64_t M, int64_t K, void* stream);

/* Y [M][N] (and S when not NULL) for Q4_0 weights x q8_0 activations.
 * K % 32 == 0; SW % 16 == 0 and SW >= K/2; WQ and XQ 16-byte aligned.
 * block_n in {8,16,32,64,128}, nb in {1,2,4,8,16}, num_warps in {1,2,4,8}; block_n == 0 picks all three for the shape.
 * mode: KOMP_MODE_*.
 * Replaces: host.gemv (src/komp/host.py:76-85) launching kernels.q4_0_gemv (src/komp/kernels.py:48-94), whose
 * argument list is (WQ, WS, XQ, XD, Y, S, N, K, SW; BLOCK_N, NB, MODE, STORE_S) (src/komp/compile.py:20-27). */
int komp_q4_0_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                   void* stream);

/* The same for TQ2_0 weights x q8_K activations.  K % 256 == 0; SW % 16 == 0 and SW >= K/4.  With block_n == 0 in
 * KOMP_MODE_DP4A, three columns run on the matrix cores when komp_gemv_mfma_plan says so (S the same, Y to f32
 * rounding).
 * Replaces: host.gemv (src/komp/host.py:76-85) launching kernels.tq2_0_gemv (src/komp/kernels.py:97-142). */
int komp_tq2_0_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                    int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                    void* stream);

/* Quantize-and-GEMV in one launch: X is f32 [M][K] (16-byte aligned); every workgroup quantizes it (q8_0 for q4_0,
 * q8_K for tq2_0) into LDS with the quantizer kernels' arithmetic, then runs the GEMV, so Y and S equal
 * komp_quant_q8_* followed by komp_*_gemv with the same block_n / nb / num_warps bit for bit (block_n == 0 plans the
 * fused launch with its own knobs, komp_gemv_auto_config with fused != 0).  When XQ is not NULL, one workgroup also writes the q8 planes
 * XQ [M][K] and XD (required with XQ), and for tq2_0 the bsums XB [M][K/16] when XB is not NULL (XB must be NULL for
 * q4_0).  Other arguments as komp_q4_0_gemv / komp_tq2_0_gemv.
 * No reference counterpart: the reference launches its quantizer and its GEMV separately (src/komp/host.py:63-85);
 * this removes one dispatch per GEMV from a decode step. */
int komp_q4_0_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                       float* XD, int16_t* XB, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb,
                       int mode, int num_warps, void* stream);
int komp_tq2_0_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                        float* XD, int16_t* XB, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb,
                        int mode, int num_warps, void* stream);

/* Several weight matrices that share one activation input, in one launch (for example Q, K and V, or gate and up,
 * stored as separate tensors): matrix i (count 1..4) has WQ[i] u8 [N[i]][SW[i]] and WS[i] i16 [N[i]][K/32] (q4_0)
 * or [N[i]][K/256] (tq2_0) and writes Y[i] f32 [M][N[i]].  Give either XQ and XD (q8 planes, as komp_q4_0_gemv /
 * komp_tq2_0_gemv) or X (f32 [M][K], quantized inside the launch as komp_q4_0_gemv_f32 / komp_tq2_0_gemv_f32), the
 * other NULL.  With the same block_n / nb / num_warps each Y[i] equals that entry run on matrix i alone, bit for bit;
 * block_n == 0 plans the launch for the matrices' rows together (komp_gemv_auto_config with N = their sum).  WQ, WS,
 * Y, N and SW are host arrays of count entries; the pointers they hold are device pointers.
 * No reference counterpart: the reference launches one matrix per kernel (src/komp/host.py:76-85); this serves the
 * per-token launch count of decoders that store their projections apart. */
int komp_q4_0_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                         const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                         int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream);
int komp_tq2_0_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                          const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                          int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream);

/* Q8_0 and IQ4_NL weights x q8_0 activations: ggml formats beyond the reference's two (its README.md:143 lists them as
 * next), on the same split planes and with the same entries and semantics as Q4_0:
 *   Q8_0    WQ u8 [N][SW] (32 int8 per block of 32, SW >= K), WS i16 [N][K/32] (f16 bits)   (ggml block_q8_0)
 *   IQ4_NL  WQ u8 [N][SW] (16 bytes per block of 32 in Q4_0's nibble order; each nibble indexes ggml's value table
 *           kvalues_iq4nl), WS i16 [N][K/32]                                              (ggml block_iq4_nl)
 * Y[m][n] = sum_b f16(d_w) * d_x * s(m, n, b) with s the exact int32 block dot of the decoded values.  The _f32
 * entries take no XB (q8_0 activations have no bsums).  No reference counterpart. */
int komp_q8_0_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                   void* stream);
int komp_iq4_nl_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                     int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                     void* stream);
int komp_q8_0_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                       float* XD, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode,
                       int num_warps, void* stream);
int komp_iq4_nl_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                         float* XD, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode,
                         int num_warps, void* stream);
int komp_q8_0_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                         const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                         int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream);
int komp_iq4_nl_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                           const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                           int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream);
int komp_q8_0_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, void* stream);
int komp_iq4_nl_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                     int64_t M, int64_t N, int64_t K, int64_t SW, void* stream);
int komp_q8_0_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream);
int komp_iq4_nl_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream);

/* Q4_K weights x q8_K activations: ggml's block_q4_K (README.md:143 lists it as a next format; no reference
 * counterpart), with TQ2_0's entries and activation planes.
 *   WQ u8 [N][SW] (128 quant bytes per 256-value block: byte 32j + l holds value 64j + l in its low nibble and
 *      64j + 32 + l in its high nibble, SW >= K/2), WS i16 [N][8 K/256], 16-byte aligned (each block's first 16
 *      bytes: f16 d, f16 dmin, 12 bytes of 6-bit sub-block scales and mins)                      (ggml block_q4_K)
 *   S i32 [M][N][K/256][2] = (sd, sm): sd = sum_i sc_i * (dot of sub-block i), sm = sum_i m_i * (sum of the
 *      activations of sub-block i), over the 8 sub-blocks of 32 values
 *   Y[m][n] = sum_b f16(d) * d_x * sd - f16(dmin) * d_x * sm                        (ggml vec_dot_q4_K_q8_K)
 * A lane loads a 32-byte group of a block per slot, so explicit knobs take nb <= 8.  komp_q4_k_gemm is the
 * matrix-core GEMM for any M (komp_q4_0_gemm's contract; S as above), and block_n == 0 in dp4a mode routes 4+
 * columns to it. */
int komp_q4_k_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                   void* stream);
int komp_q4_k_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                       float* XD, int16_t* XB, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb,
                       int mode, int num_warps, void* stream);
int komp_q4_k_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                         const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                         int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream);
int komp_q4_k_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, void* stream);
int komp_q4_k_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream);

/* The plan that block_n == 0 selects for a GEMV shape on the current device; fmt 0 = q4_0, 1 = tq2_0, 2 = q8_0,
 * 3 = iq4_nl, 4 = q4_k; fused != 0 for
 * komp_q4_0_gemv_f32 / komp_tq2_0_gemv_f32; mode as in the GEMV entries; M the activation columns.  block_n receives
 * the rows per workgroup, nb the 16-byte weight chunks each lane loads per row per K step, num_warps the waves per
 * workgroup, and (when not NULL) lanes_per_row the lanes that share a row and passes the row groups each wave walks
 * in sequence.  The explicit knobs map (block_n, nb, num_warps) to lanes_per_row = 64 / min(block_n / num_warps, 16)
 * and passes = (block_n / num_warps) / min(block_n / num_warps, 16); an auto plan with other values, or with
 * block_n / num_warps outside the knob sets (one workgroup of ceil(N / CUs) rows per CU, up to 16 waves, for small
 * single-column GEMVs), has no explicit knob equivalent.  (Explicit knobs of unfused single Q4_0 / IQ4_NL columns
 * whose block_n-row programs hold no more waves than the device has CUs launch each wave as a workgroup of its own:
 * the same rows, lanes and K steps a wave, the same results.)
 * No reference counterpart: the reference always takes the knobs from its caller. */
int komp_gemv_auto_config(int fmt, int fused, int mode, int64_t M, int64_t N, int64_t K, int* block_n, int* nb,
                          int* num_warps, int* lanes_per_row, int* passes);

/* Y [M][N] (and S when not NULL) as komp_q4_0_gemv / komp_tq2_0_gemv compute them, for any M, on the matrix cores
 * (v_mfma_i32_16x16x32_i8 / v_mfma_i32_16x16x64_i8): each workgroup reads its weight rows once for up to 64
 * activation columns, where the GEMVs read them once per 3.  S is bit-identical to the GEMVs'; Y agrees to f32
 * rounding (the f32 sums run in another order).  Arguments and alignment as komp_q4_0_gemv / komp_tq2_0_gemv without
 * the knobs; also 64*K and 32*SW must be below 2^31 and the 16 or 32 rows of WS a workgroup stages must fit in LDS
 * (komp_gemm_plan says whether a shape qualifies).  komp_q4_0_gemv / komp_tq2_0_gemv with block_n == 0 and
 * KOMP_MODE_DP4A run this kernel for M >= 4 when the shape qualifies.
 * No reference counterpart: the reference launches its GEMV once per column (grid (cdiv(N, BLOCK_N), M),
 * src/komp/kernels.py:50); this serves batched decode, where M columns share every weight byte. */
int komp_q4_0_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, void* stream);
int komp_tq2_0_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                    int64_t M, int64_t N, int64_t K, int64_t SW, void* stream);

/* The matrix-core GEMM's plan for a shape on the current device (fmt as komp_gemv_auto_config): weight rows and activation
 * columns per workgroup, waves per workgroup.  Returns KOMP_EINVAL when the shape is past the kernel's limits.
 * No reference counterpart. */
int komp_gemm_plan(int fmt, int64_t M, int64_t N, int64_t K, int64_t SW, int* rows_per_wg, int* cols_per_wg,
                   int* waves);

/* Whether komp_tq2_0_gemv with block_n == 0 runs the matrix-core GEMV for this call (fused 0 / 1, mode as the GEMVs):
 * TQ2_0, KOMP_MODE_DP4A, 3 columns, more than 8 rows a CU, rows of at most 64 blocks, SW a multiple of 16, q8_K
 * activations in (f32 in: from 4 row tiles a CU on).  Returns 1 and its workgroup's rows (spread evenly over the
 * CUs, at most 16, or 32 in two tiles) and waves when it does, 0 (and zeros) when the call runs on the GEMV kernels, KOMP_EINVAL on a bad
 * argument.  That kernel computes S bit-identical to the GEMVs' and Y to f32 rounding (its f32 sums run in another
 * order): the activations are the A operand of v_mfma_i32_16x16x64_i8 and 16 weight rows its B operand, so the VALU
 * work per weight does not grow with the columns.
 * No reference counterpart: the reference runs one program per column (src/komp/kernels.py:50). */
int komp_gemv_mfma_plan(int fmt, int fused, int mode, int64_t M, int64_t N, int64_t K, int64_t SW, int* rows_per_wg,
                        int* waves);

/* ggml block bytes -> KURN's split planes on the device.  W: N rows of K/32 Q4_0 blocks (18 bytes: f16 d, 16 quant
 * bytes) or K/256 TQ2_0 blocks (66 bytes: 64 quant bytes, f16 d), contiguous, 4-byte aligned.  Writes WQ u8 [N][SW]
 * (16-byte aligned, SW % 16 == 0, SW >= K/2 resp. K/4; the padding past a row's quant bytes is left as it was) and
 * WS i16 [N][K/blk] (2-byte aligned); the bytes equal the reference's host split.
 * Replaces: host.split (src/komp/host.py:16-22), which does this with numpy on the host. */
int komp_q4_0_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream);
int komp_tq2_0_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream);

/* OUT[i] = dp4a(A[i], B[i], C[i]) for i < n; mode KOMP_MODE_DP4A (hardware) or KOMP_MODE_DP4A_EMU.
 * Replaces: kernels.dp4a_probe (src/komp/kernels.py:145-149). */
int komp_dp4a_probe(const int32_t* A, const int32_t* B, const int32_t* C, int32_t* OUT, int64_t n, int mode,
                    void* stream);

/* Reads the BYTES of SRC once (streaming 16-byte buffer loads, 2048 per 512-thread workgroup) and writes the XOR of each
 * wave's 512 dwords to OUT[wave], 8 * ceil(BYTES / 32768) words: the cost of moving the bytes alone, the floor a GEMV
 * over as many bytes is compared with.  BYTES % 16 == 0, SRC 16-byte and OUT 4-byte aligned.
 * No reference counterpart: a measurement probe (bench.py reports every GEMV shape against it). */
int komp_stream_read(const void* SRC, int64_t bytes, uint32_t* OUT, void* stream);

/* [R][16] Q4_0 quant bytes -> [R][32] int32 values.  Replaces: kernels.q4_0_decode (src/komp/kernels.py:152-157). */
int komp_q4_0_decode(const uint8_t* WQ, int32_t* OUT, int64_t R, void* stream);

/* [NBLK][64] TQ2_0 quant bytes -> [NBLK][256] int32 values.  Replaces: kernels.tq2_0_decode (src/komp/kernels.py:160-170). */
int komp_tq2_0_decode(const uint8_t* WQ, int32_t* OUT, int64_t nblk, void* stream);

/* Dispatch timing for the tuning harness (no reference counterpart; the reference was never timed).
 * Between komp_timing_begin() and komp_timing_end(), every launch made by this library on the calling process is
 * issued with hipExtLaunchKernel start/stop events, which the runtime stamps with the dispatch's own begin and end.
 * komp_timing_end() waits for those events and returns, per kernel kind, the summed dispatch time in milliseconds and
 * the dispatch count.  Kinds: 0 quant_q8_0, 1 quant_q8_K, 2 q4_0 GEMV / GEMM, 3 tq2_0 GEMV / GEMM, 4 probes and
 * weight splits, 5 q8_0 GEMV / GEMM, 6 iq4_nl GEMV / GEMM, 7 q4_k GEMV (arrays of length 8).
 * max_dispatches bounds the events created. */
#define KOMP_TIMING_KINDS 8
int komp_timing_begin(int64_t max_dispatches);
int komp_timing_end(double* ms, int64_t* count);

/* In-kernel wave stamps for the tuning harness (no reference counterpart; the reference was never timed): the span of
 * a kernel inside a HIP graph, from its first wave's entry to its last wave's stored outputs, which no event can see.
 * Between komp_stamps_begin() and komp_stamps_end(), every TQ2_0 GEMV launch in dp4a mode (fused or not) whose plan
 * reads its rows in one pass and one K step, from a single matrix (the decode shapes' plans), runs an instantiation
 * of the same kernel that reads the device's constant-rate real-time counter in every wave at four points: entry,
 * the staged activations published to the workgroup, the last weight chunk's dot issued, and the wave's outputs
 * stored (the stores complete).  Other launches run as usual and record nothing, and so does a launch that no longer
 * fits in BUF.  BUF (device memory, 16-byte aligned, WORDS uint32 words) receives per stamped launch, at the next
 * 16-byte boundary: a header {0x4B535450, waves of the grid, N, K}, then {entry, staged, dots, stored} per wave (the
 * counter's low 32 bits), wave w of workgroup g at index g * (waves per workgroup) + w.  A launch captured into a HIP
 * graph keeps its records' place, and each replay rewrites them.  komp_stamps_end() returns the words used and the
 * counter's rate in kHz (hipDeviceAttributeWallClockRate). */
int komp_stamps_begin(uint32_t* buf, int64_t words);
int komp_stamps_end(int64_t* words_used, int* clock_khz);

/* Writes the same real-time counter (64 bits) to OUT[0] (device, 8-byte aligned) when `stream` reaches the call: a
 * one-lane kernel that marks a point of the stream's work, where events cannot be recorded (inside a HIP graph; the
 * benchmark times its K decode steps between two such marks of one graph).  komp_clock_khz gives the counter's rate.
 * No reference counterpart (a measurement probe). */
int komp_clock(uint64_t* OUT, void* stream);
int komp_clock_khz(int* khz);

#ifdef __cplusplus
}
#endif

#endif /* KOMP_ABI_H */
