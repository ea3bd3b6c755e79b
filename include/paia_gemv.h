/* paia_gemv.h -- C ABI of libpaia_gemv.so, the gfx950 (MI355X) HIP build of the PAIA M=1 GEMV family.
 *
 * Drop-in for the reference's ctypes-loaded libpaia_gemv.so (Bejaine/PAIA-Project, src/paia_gemv/): the first eleven
 * entry points keep the reference's names, argument order, argument meaning, alignment contract and return codes.
 * The rest are additions for the BASELINE configurations (bias epilogue, asymmetric INT4, on-device dequantisation).
 *
 * Conventions (all entry points, as src/paia_gemv/gemv_quant.cu:2 and gemv_bf16.cu:44-47):
 *   return 0 ok; -1 bad variant index; -2 bad shape or alignment; > 0 a hipError_t reported after the launch.
 *   All pointers are caller-owned device memory. The library allocates nothing, keeps no handles, never
 *   synchronises, and launches on `stream` (a hipStream_t; NULL = the null stream), so calls are graph-capturable.
 *   x, y and bias are bf16 bit patterns; N, K are ints with size_t offsets inside.
 *   y[n] = bf16_round_to_nearest_even( sum_k deq(W[n,k]) * x[k] (+ bias[n]) ), fp32 accumulation.
 *
 * K: every K of the alignment rules runs, as in the reference. x is staged in 64 KiB of LDS per block up to BF16 and
 *   FP8 K <= 32768, INT4 K <= 30720 (split-K variants (H=1) also keep one round of partial sums there: BF16
 *   K <= 32256, FP8 K <= 31744); beyond that the call runs an x-from-global kernel (x read with each item's weights,
 *   split-K over 8 waves) whatever the variant, slower but with the same contract. All Llama-3.1-8B / Qwen2.5-7B
 *   shapes stage x.
 * INT4 x: any finite bf16 activations, as in the reference. The M=1 kernels that stage x read the nibbles either
 *   as bf16 subnormals against x scaled by a power of two (2^64 when the row's largest |x| lies in [2^-20, 2^64),
 *   else a power picked from that largest |x|, so every staged value and product stays a normal number) or, on
 *   launches with few weight loads per wave, as bf16 (128 + q) against unscaled x.
 */
#ifndef PAIA_GEMV_H
#define PAIA_GEMV_H

#ifdef __cplusplus
extern "C" {
#endif

#define PAIA_API __attribute__((visibility("default")))

/* ---- BF16: W bf16 [N][K] row-major. K % 8 == 0; W, x, y 16-byte aligned. ---------------------------------- */

/* replaces src/paia_gemv/gemv_bf16.cu:38 */
PAIA_API int paia_gemv_bf16_variant_count(void);
/* replaces src/paia_gemv/gemv_bf16.cu:41-45. Knobs (gfx950 meaning): R rows per wave, U 16-byte loads per row per
 * batch, W waves per block, S nontemporal weight loads, H split-K across the waves of a block. */
PAIA_API int paia_gemv_bf16_variant_info(int v, int* R, int* U, int* W, int* S, int* H);
/* replaces src/paia_gemv/gemv_bf16.cu:48-53 */
PAIA_API int paia_gemv_bf16(const void* W, const void* x, void* y, int N, int K, int variant, void* stream);
/* no reference counterpart (BASELINE Qwen qkv bias epilogue): bias bf16 [N], 2-byte aligned, or NULL */
PAIA_API int paia_gemv_bf16_bias(const void* W, const void* x, const void* bias, void* y, int N, int K, int variant,
                                 void* stream);

/* ---- FP8 W8A16: Wq e4m3fn [N][K], scale fp32 [N]. K % 16 == 0; Wq, x 16-byte, scale 4-byte, y 2-byte aligned. -- */

/* replaces src/paia_gemv/gemv_quant.cu:61 */
PAIA_API int paia_gemv_fp8_variant_count(void);
/* replaces src/paia_gemv/gemv_quant.cu:62 */
PAIA_API int paia_gemv_fp8_variant_info(int v, int* R, int* U, int* W, int* H);
/* replaces src/paia_gemv/gemv_quant.cu:64-68 */
PAIA_API int paia_gemv_fp8(const void* Wq, const void* scale, const void* x, void* y, int N, int K, int variant,
                           void* stream);
/* no reference counterpart (bias epilogue for the FP8 Qwen qkv config): bias bf16 [N] or NULL */
PAIA_API int paia_gemv_fp8_bias(const void* Wq, const void* scale, const void* x, const void* bias, void* y, int N,
                                int K, int variant, void* stream);

/* ---- INT4 W4A16 g128, reference format: Wq [N][K/2] (byte j = weights 2j low nibble, 2j+1 high nibble, i.e. 8 per
 *      int32 along K), zero point 8, scales fp16 [N][K/128]. K % 128 == 0; Wq, x 16-byte, scales, y 2-byte. ----- */

/* replaces src/paia_gemv/gemv_quant.cu:70 */
PAIA_API int paia_gemv_int4_variant_count(void);
/* replaces src/paia_gemv/gemv_quant.cu:71 */
PAIA_API int paia_gemv_int4_variant_info(int v, int* R, int* U, int* W, int* H);
/* replaces src/paia_gemv/gemv_quant.cu:73-77 */
PAIA_API int paia_gemv_int4(const void* Wq, const void* scales, const void* x, void* y, int N, int K, int variant,
                            void* stream);
/* replaces src/paia_gemv/gemv_quant.cu:80-85 (the naive K1 control) */
PAIA_API int paia_gemv_int4_naive(const void* Wq, const void* scales, const void* x, void* y, int N, int K,
                                  void* stream);
/* replaces src/paia_gemv/gemv_quant.cu:88-97 (the unfused control): scratch_bf16 is caller-owned, 2*N*K bytes,
 * 16-byte aligned; y must satisfy the BF16 contract (16-byte aligned). */
PAIA_API int paia_gemv_int4_unfused(const void* Wq, const void* scales, const void* x, void* y, void* scratch_bf16,
                                    int N, int K, void* stream);

/* No reference counterpart: for callers that cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc), paia_gemv_int4_unfused without the caller's workspace. The dequantised
 * bf16 rows go to a 32 MiB static device buffer of the library (one per GPU, held until the process ends), slice by
 * slice of at most 32 MiB / (2K) rows (a multiple of 8), each slice's BF16 GEMV right after its dequantisation; the
 * result equals paia_gemv_int4_unfused's bit for bit. Allocates nothing (the buffer's device address is looked up
 * once per device, on the first call there). Returns -2 also when 8 rows do not fit the buffer (K > 2097152). Calls
 * that overlap on one GPU (other streams, other threads) share the buffer and race: serialise them. */
PAIA_API int paia_gemv_int4_unfused_noalloc(const void* Wq, const void* scales, const void* x, void* y, int N, int K,
                                            void* stream);

/* ---- INT4 W4A16 g128, asymmetric format (no reference counterpart; BASELINE INT4 configs): q in 0..15 packed as
 *      above, scales bf16 [N][G] (G = K/128), zeros [N][ceil(G/2)] bytes (group 2j low nibble, 2j+1 high nibble),
 *      dequant (q - z) * s; optional bias bf16 [N] (or NULL). Uses the paia_gemv_int4 variant table. --------- */
PAIA_API int paia_gemv_int4_zp(const void* Wq, const void* scales, const void* zeros, const void* x, const void* bias,
                               void* y, int N, int K, int variant, void* stream);

/* ---- on-device dequantisation to fp32 [N][K] (no reference C symbol; the values of src/paia_gemv/quant.py:16-17,
 *      34-38 and quant_host.h:82-85,106-111). out 16-byte aligned. ---------------------------------------------- */
PAIA_API int paia_dequant_fp8(const void* Wq, const void* scale, void* out, int N, int K, void* stream);
PAIA_API int paia_dequant_int4(const void* Wq, const void* scales, void* out, int N, int K, void* stream);
PAIA_API int paia_dequant_int4_zp(const void* Wq, const void* scales, const void* zeros, void* out, int N, int K,
                                  void* stream);

/* ---- on-device quantizers from fp32 W [N][K] row-major (no reference C symbol: the reference quantizes with torch,
 *      src/paia_gemv/quant.py:8-31; same values as quant.py / quant_host.h:74-106). W 16-byte aligned. ------------ */
/* q e4m3fn [N][K] (16-byte aligned), scale fp32 [N]: scale = amax/448 (1 for a zero row), q = e4m3_rn(clamp(w/scale,
 * +-448)). K % 16 == 0. Replaces torch quantize_fp8_rowwise (src/paia_gemv/quant.py:8-13). */
PAIA_API int paia_quantize_fp8_rowwise(const void* W, void* q, void* scale, int N, int K, void* stream);
/* packed [N][K/2] (16-byte aligned), scales fp16 [N][K/128]: s = f16(amax/7) (1 for a zero group, 1 where it
 * underflows), n = clamp(rint(w/s), -7, 7) + 8. K % 128 == 0. Replaces torch quantize_int4_g128 (quant.py:20-31). */
PAIA_API int paia_quantize_int4_g128(const void* W, void* packed, void* scales, int N, int K, void* stream);
/* no reference counterpart (asymmetric INT4 of the BASELINE configs): per group of 128, lo = min(0, min w),
 * hi = max(0, max w), s = bf16((hi - lo)/15) (1 if 0), z = clamp(rint(-lo/s), 0, 15), q = clamp(rint(w/s) + z, 0, 15);
 * packed [N][K/2], scales bf16 [N][G], zeros [N][ceil(G/2)] (group 2j low nibble). K % 128 == 0. */
PAIA_API int paia_quantize_int4_zp_g128(const void* W, void* packed, void* scales, void* zeros, int N, int K,
                                        void* stream);

/* no reference counterpart (the reference picks variants in Python from src/tuned/<platform>.json,
 * paia-bench/bench/ops/ours_bf16.py:32-38): the library's per-shape variant for kind 0 BF16, 1 FP8, 2 INT4 reference
 * format, 3 INT4 asymmetric (an index of the paia_gemv_int4 table). Always returns a valid index of that table. */
PAIA_API int paia_gemv_pick_variant(int kind, int N, int K);
/* no reference counterpart (for profilers and tools that name the kernel a call runs): which kernel a launch of
 * `variant` of kind 0 BF16, 1 FP8, 2 INT4 reference format, 3 INT4 asymmetric runs at (N, K): 0 gemv_kernel,
 * 1 gemv_kernel43 (INT4 launches whose waves make at most 7 weight loads: the bf16 (128 + q) decode), 2 gemv_kernel_xg
 * (K beyond the LDS staging), 3 gemv_kernel_dr and 4 gemv_kernel43_dr (0 and 1 for row-parallel launches whose waves
 * take at most two items: the walk ends in a drain); -1 bad kind or variant, -2 bad shape. Launches nothing. */
PAIA_API int paia_gemv_launch_kind(int kind, int N, int K, int variant);

/* ---- small batch: M = 1..16 activation rows (matrix-core kernel, row-streaming kernel on the M = 1 design, and the
 * M = 1 GEMV itself at M = 1; the library picks per shape and M). No reference symbol: the reference's kernels are
 * M = 1 only and M = 1..16 is its open item (src/README.md:118, swept by paia-bench/configs/shapes.yaml:63-64).
 * x bf16 [M][K] row-major (16-byte aligned), y bf16 [M][N] row-major (2-byte aligned); the weight operands, their
 * alignment and the K rules are those of the M = 1 entry point of the same format. bias bf16 [N] or NULL.
 * kind: 0 BF16, 1 FP8, 2 INT4 reference format, 3 INT4 asymmetric. variant < 0 = paia_gemv_batch_pick_variant's.
 * Knobs: P tiles of 16 rows per wave, U k-blocks of 128 columns in flight per wave, W waves per block, S waves
 * sharing a tile along K, X = 0 x staged in LDS per K-chunk of up to 64 KiB / 1 x loaded with the weights / 2 x
 * staged as for 0 in K-chunks of up to 80 KiB (or the device's per-block LDS if less). P = 0 marks a
 * row-streaming variant (the M = 1 kernel's weight stream with one accumulator per activation row): U 1-KiB chunks
 * per item, W waves per block, S weight rows per wave, and X the one M (2-6; BF16 and FP8 2-8) it serves. The last variant of
 * each table (P = U = W = S = 0, X = 1) is the M = 1 GEMV itself with paia_gemv_pick_variant's choice (M = 1 only;
 * the batch alignment rules hold for it, y included). Returns 0, -1 bad variant, -2 bad shape/alignment (or, X = 0
 * or 2, S*M*U too large for the LDS chunk; or, P = 0, another M or M copies of the staged x beyond the device's per-block
 * LDS, 160 KiB on MI355X), > 0
 * hipError_t. */
PAIA_API int paia_gemv_batch_variant_count(int kind);
PAIA_API int paia_gemv_batch_variant_info(int kind, int v, int* P, int* U, int* W, int* S, int* X);
PAIA_API int paia_gemv_batch_pick_variant(int kind, int M, int N, int K);
PAIA_API int paia_gemv_batch_bf16(const void* W, const void* x, const void* bias, void* y, int M, int N, int K,
                                  int variant, void* stream);
PAIA_API int paia_gemv_batch_fp8(const void* Wq, const void* scale, const void* x, const void* bias, void* y, int M,
                                 int N, int K, int variant, void* stream);
PAIA_API int paia_gemv_batch_int4(const void* Wq, const void* scales, const void* x, void* y, int M, int N, int K,
                                  int variant, void* stream);
PAIA_API int paia_gemv_batch_int4_zp(const void* Wq, const void* scales, const void* zeros, const void* x,
                                     const void* bias, void* y, int M, int N, int K, int variant, void* stream);

/* no reference counterpart: a human-readable build tag */
PAIA_API const char* paia_gemv_build_info(void);

#ifdef __cplusplus
}
#endif
#endif
