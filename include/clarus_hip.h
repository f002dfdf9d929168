/*
 * clarus_hip.h - C ABI of libclarus_hip.so, the MI355X (gfx950) kernels behind the `hip`
 * operator backend of clarus.
 *
 * The reference has no native FFI on this path: its Python adapter
 * (python/clarus/ops/triton_cuda.py) calls Triton launch wrappers. Each entry point below
 * replaces one of those wrappers (cited per function); the Python adapter
 * clarus_amd/hip_ops.py binds them with ctypes. Conventions:
 *
 *   - Plain device pointers, int64 sizes and strides in ELEMENTS, dtype codes, and an opaque
 *     stream (a hipStream_t passed as void*; NULL = the null stream).
 *   - The library owns no device memory. Scratch space (split-K partials) is passed in.
 *   - Every call validates its arguments before launching anything and returns 0 on success,
 *     CLARUS_EINVAL for arguments the kernels do not handle, or CLARUS_ELAUNCH when the HIP
 *     launch failed. clarus_hip_last_error() describes the last failure of the calling thread.
 *   - No call synchronizes, allocates or loads modules, so all of them may be recorded into a
 *     HIP graph.
 *   - Activations are NHWC. A "pixel stride" is the element distance between consecutive
 *     pixels, which lets an operand be a channel slice of a wider NHWC buffer.
 */
#ifndef CLARUS_HIP_H
#define CLARUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CLARUS_HIP_ABI_VERSION 2

/* return codes */
#define CLARUS_OK 0
#define CLARUS_EINVAL 1
#define CLARUS_ELAUNCH 2

/* element types */
#define CLARUS_F32 0
#define CLARUS_BF16 1

/* prologue on A, applied in fp32 before the product (python/clarus/kernels/gemm.py:5-10) */
#define CLARUS_PRO_NONE 0  /* a                                                   */
#define CLARUS_PRO_LN 1    /* (a - mean) * rstd over the K channels (eps ln_eps)   */
#define CLARUS_PRO_MUL 2   /* a * S[clamp(y - pt), clamp(x - pl), k] (TLC map)      */
#define CLARUS_PRO_RMS 3   /* a * rsqrt(mean(a^2) + eps)                            */
#define CLARUS_PRO_LNMUL 5 /* ((a - mean) * rstd * lnw[k] + lnb[k]) * act(m2[p, k]) */
/* or-ed into pro (LN / RMS / TLC map with bf16 A and W): the prologue output may be rounded once
   to bf16 (RNE) before the product, the reference GPU path's arithmetic (kernels/gemm.py:164-186);
   the ring streaming kernel (K <= 128) does so, the other kernels keep hi + lo bf16 pairs */
#define CLARUS_PRO_ROUND 0x100

/* A addressing */
#define CLARUS_A_ROWS 0  /* row p at a + p * lda                                    */
#define CLARUS_A_S2D 1   /* 2x2 stride-2 conv: K = (dy, dx, cin), input [*, h, w, K/4] */

/* C addressing */
#define CLARUS_C_ROWS 0    /* out[p * ldc + n]                                      */
#define CLARUS_C_SHUFFLE 1 /* PixelShuffle(2): N = (dy, dx, c'), output [*, 2h, 2w, N/4] */
#define CLARUS_C_NCHW 2    /* out[((img * N + n) * h + y) * w + x] (conv only)      */

/* activations */
#define CLARUS_ACT_NONE 0
#define CLARUS_ACT_GELU 1  /* exact erf GELU                                        */
#define CLARUS_ACT_LRELU 2 /* LeakyReLU(slope)                                      */

/*
 * Fused NHWC GEMM:  out[p, n] = epilogue( prologue(A)[p, :] . W[:, n] ), fp32 accumulation.
 *
 * W is passed TRANSPOSED, wt[n_cols][k] with k contiguous (n_cols = 2n when gate), in bf16
 * or fp32. Operand handling (chosen by the library from the dtypes and the prologue):
 *   bf16 A, no prologue, bf16 W  -> bf16 MFMA (products exact in fp32)
 *   fp32 A or a prologue, bf16 W -> A split into bf16 hi + lo, two bf16 MFMAs
 *   any A, fp32 W                -> fp32 MFMA
 * Epilogue order (python/clarus/ops/torch_ref.py:119-131):
 *   + bias[n] (and bias[n + N] on the gate half) -> SimpleGate o1 * o2 -> act -> * scale[n]
 *   -> * out_scale -> + residual -> cast to c_dtype.
 * batch > 1 runs `batch` independent GEMMs of m rows (linear_per_image) using the batch strides.
 * out may alias residual exactly (same pointer and strides).
 */
typedef struct ClarusGemmArgs {
  const void* a;
  const void* wt;
  void* c;
  const float* bias;  /* [n] or [2n] with gate; NULL for none        */
  const float* scale; /* [n]; NULL for none                          */
  const void* res;    /* residual addressed like the output; NULL    */
  const void* small;  /* PRO_MUL map [batch, oh, ow, k]              */
  const void* m2;     /* PRO_LNMUL multiplier rows, pixel stride ldm2 */
  const float* lnw;   /* PRO_LNMUL LayerNorm affine [k]              */
  const float* lnb;
  float* stats;       /* optional scratch, 2 * m floats (batch 1): with PRO_LN / PRO_RMS /
                         PRO_LNMUL and K > 128 the row statistics are computed into it by a
                         separate pass (one read of A) instead of inside every column tile */
  int64_t m;          /* rows (output pixels) per batch entry         */
  int64_t n;          /* output channels                              */
  int64_t k;          /* reduction length                             */
  int64_t batch;
  int64_t lda, ldc, ldr, ldm2;       /* pixel strides (elements)        */
  int64_t a_bstride, w_bstride, c_bstride, r_bstride; /* batch strides */
  int32_t a_dtype, w_dtype, c_dtype, r_dtype, s_dtype, m2_dtype;
  int32_t h, w;       /* A_S2D: input size; C_SHUFFLE: input size; PRO_MUL: image size */
  int32_t oh, ow, pt, pl; /* PRO_MUL map geometry (torch_ref.py:18-41)                  */
  int32_t pro, a_mode, c_mode, gate, act, m2_act;
  float ln_eps, out_scale, slope;
  int32_t tile;       /* 0 = library's choice; else a kernel / tile id for sweeps: 1-7 tiled
                         shapes, 8 / 9 W-resident streaming (4 / 8 channel blocks), 10 pipelined
                         LDS tile, 11 DMA-pipelined tile (bf16 A, no prologue, K % 32 == 0),
                         13 DMA-pipelined 32x32-MFMA tile (bf16 A, no prologue, K % 64 == 0),
                         14 / 15 the same with 256 / 128 pixels x 256 channels per tile,
                         16 / 17 streaming with a per-wave LDS ring (K <= 128 bf16 / 64 fp32;
                         17: 4 channel blocks per workgroup), 18 W-slice (bf16 A and W, no
                         prologue / gate / act / residual, K = 128 / 256 / 512, N % 64 == 0) */
} ClarusGemmArgs;

/* replaces kernels/gemm.py:353-400 fused_gemm and :403-429 _gemm_wide */
int clarus_hip_gemm(const ClarusGemmArgs* args, void* stream);

/*
 * clarus_hip_gemm for plain bf16 rows (a_mode rows, pro none, batch 1, c_mode rows) with bf16 W,
 * K = 256, 512 or 1024 and W^T rows (n, or 2 n with gate) a multiple of 512, with W^T
 * also passed packed. pro may also be CLARUS_PRO_LN / CLARUS_PRO_RMS (ln_eps) without a residual
 * at K <= 512, on bf16 or fp32 rows, or CLARUS_PRO_MUL (bf16 rows and map; small, s_dtype, h, w,
 * oh, ow, pt, pl as for clarus_hip_gemm, m a multiple of h w) with a residual at K <= 512: the
 * result is bit for bit clarus_hip_rows_prologue's rows (rounded once to bf16) through this entry
 * point, in one launch.
 * wp holds W^T in the fragment order of clarus_hip_gemm_ln_gemm's w2p (K
 * columns instead of 512: for pass P, wave w, 16-k step s (0 .. K / 16 - 1), block b, lane l, the
 * 8 values W^T[row(P, 64 w + 32 b + l % 32)][16 s + 8 (l / 32) + e], with gate2 = gate).
 * args->wt is not read. Epilogue as clarus_hip_gemm: bias (SimpleGate), act (none / GELU /
 * leaky ReLU), scale * out_scale, bf16 / fp32 residual, bf16 / fp32 output.
 * replaces kernels/gemm.py:353-400 fused_gemm for those shapes (the weight packed once per
 * weight by the host, as the reference's ops cache their transposed weights)
 */
int clarus_hip_gemm_wp(const ClarusGemmArgs* args, const void* wp, void* stream);

/*
 * clarus_hip_gemm for plain bf16 rows (a_mode rows, pro none, batch 1, c_mode rows) with bf16 W,
 * K = 128 or 256 and N a multiple of 16, on a persistent kernel that keeps each workgroup's
 * 512-row W^T pass in registers for all of its pixel tiles. pro may also be CLARUS_PRO_LN /
 * CLARUS_PRO_RMS (ln_eps) without a residual, or CLARUS_PRO_MUL without gate (bf16 map; small,
 * s_dtype, h, w, oh, ow, pt, pl as for clarus_hip_gemm; at K = 256 n <= 256): each A tile's rows are
 * normalised / multiplied in LDS before its products, bit for bit what clarus_hip_rows_prologue
 * would have written. wp is W^T packed as for
 * clarus_hip_gemm_wp after padding: with gate each half of W^T padded to a multiple of 256 rows
 * (n2w = 2 * 256 * ceil(n / 256)), without it W^T padded to a multiple of 512 rows, the padding
 * zero. A residual (bf16 / fp32) needs n a multiple of 256 with gate, n = 256 without it, or a
 * bf16 residual with n = 128 or a multiple of 512. args->wt is not read. Epilogue as clarus_hip_gemm.
 * replaces kernels/gemm.py:353-400 fused_gemm for those shapes (the weight packed once per
 * weight by the host, as the reference's ops cache their transposed weights)
 */
int clarus_hip_gemm_wr(const ClarusGemmArgs* args, const void* wp, void* stream);

/*
 * Fused pointwise feed-forward on dense NHWC rows x [m][c] (c = 32 or 64, or 128 with bf16), one kernel:
 *   u   = SimpleGate(pro(x) . w1 + b1)          w1 [c][2c]: the product of the two c-halves
 *   out = x + (u . w2 + b2) * scale * out_scale  w2 [c][c]
 * pro = CLARUS_PRO_NONE, CLARUS_PRO_LN or CLARUS_PRO_RMS (no affine, eps ln_eps). dtype (bf16 or
 * fp32) is the type of x, out and both weights; u is rounded to it as a separate GEMM would store
 * it; with bf16 the normalised row is rounded once to bf16 before the product. b1 [2c], b2 [c],
 * scale [c]: fp32 or null. out must not overlap x. The weights are passed packed:
 *   w1p[T][s][l][i]  = w1[16 s + 8 (l / 32) + i][32 T + l % 32]       T < 2c/32, s < c/16, l < 64, i < 8
 *   w2p[T2][T][l][j] = w2[32 T + 8 (j / 4) + 4 (l / 32) + j % 4][o(T2, l % 32)]     T2, T < c/32, j < 16
 *   o(T2, r) = 32 T2 + 16 (r / 16) + 8 ((r / 4) % 2) + 4 ((r / 8) % 2) + r % 4
 * (the host packs each weight once, as the reference's ops cache their transposed weights).
 * No counterpart in the reference: it composes two `linear` calls (ops/torch_ref.py:103-130 /
 * ops/triton_cuda.py:84-112), conv4 -> conv5 of the NAFNet block (models/nafnet/__init__.py:
 * 159-161) and the pointwise benchmark chain, for hosts that run them back to back.
 */
int clarus_hip_ffn(const void* x, void* out, int dtype, const void* w1p, const float* b1, const void* w2p,
                   const float* b2, const float* scale, int64_t m, int64_t c, int pro, float ln_eps,
                   float out_scale, void* stream);

/*
 * The first half of a NAFNet block at width 64 as one kernel, for bf16 NHWC x [n][h][w][64]:
 *   t   = LN(x) . w1 + b1                 w1 [64][128] (linear layout), t rounded to bf16
 *   out = SimpleGate(dwconv3x3(t) + dwb)  taps [9][128] fp32 (tap = 3 ky + kx), 'same' zero
 *                                         padding, out [n][h][w][64] bf16
 * The LayerNorm (no affine, eps ln_eps) enters the product as bf16 hi + lo pairs; b1, dwb: fp32
 * [128] or null. out must not overlap x; n h w 64 bf16 elements must fit 2 GiB. w1p is w1 packed:
 *   w1p[T][s][l][i] = w1[16 s + 8 (l / 32) + i][o(T, l % 32)]   T < 4, s < 4, l < 64, i < 8
 *   o(T, r) = 32 T + 16 (r / 16) + 8 ((r / 4) % 2) + 4 ((r / 8) % 2) + r % 4
 * No counterpart in the reference: it composes `linear` (ln=True) and `dwconv` (gate=True),
 * models/nafnet/__init__.py:155-156 (ops/triton_cuda.py:84-112 and the dwconv op), for hosts
 * that run them back to back.
 */
int clarus_hip_ln_gemm_dwconv(const void* x, void* out, const void* w1p, const float* b1, const float* taps,
                              const float* dwb, int64_t n, int64_t h, int64_t w, int64_t c, float ln_eps,
                              void* stream);

/*
 * Prologue pass of the split-operand GEMM path. Applies the prologue of args (pro = LN, RMS
 * or the TLC map multiply, with its eps / map geometry; a, lda, m, k, a_dtype) to every row in
 * fp32 and writes out[r] = [hi(0..k) | lo(0..k)], bf16, 2k elements per row, hi = bf16(v),
 * lo = bf16(v - hi). clarus_hip_gemm on out with k' = 2k and the weights duplicated along k
 * ([W | W]) then equals the prologue GEMM to within 2^-16 relative per operand element.
 * batch must be 1 (images folded into m); k a multiple of 8, at most 2048; a and out 16-byte
 * aligned, out dense [m][2k].
 * replaces kernels/spatial.py:312 ln_rows and mul_small, the separate prologue passes of
 * ops/triton_cuda.py:101-108 (which round the prologue's output to the compute dtype instead)
 */
int clarus_hip_rows_split(const ClarusGemmArgs* args, void* out, void* stream);

/*
 * Prologue pass rounded once: the same prologue as clarus_hip_rows_split, written as one bf16
 * row of k elements, out[r] = bf16(v) (round to nearest even), out dense [m][k]. A plain bf16
 * clarus_hip_gemm on out with the original k then computes what the reference's GPU path
 * computes for a bf16 model: the prologue output rounded to the operand dtype, then a
 * tensor-core product with fp32 accumulation. Same argument rules as clarus_hip_rows_split;
 * both also take pro = none on fp32 rows (a plain conversion, the reference's fp32 A operand
 * rounded to the weights' dtype, kernels/gemm.py:187-193).
 * replaces kernels/spatial.py:312 ln_rows (out_dtype = the compute dtype) and :342 mul_small,
 * as called at ops/triton_cuda.py:104-110
 */
int clarus_hip_rows_prologue(const ClarusGemmArgs* args, void* out, void* stream);

/*
 * clarus_hip_gemm (plain bf16 rows: no prologue, gate, activation, batch or pixel shuffle,
 * N = 512, K % 64 == 0; bias, scale, residual and the output as in clarus_hip_gemm) whose
 * epilogue also writes ln_out[m][512] (bf16, dense): the output rows normalised with two-pass
 * LayerNorm (rms = 0) or RMS norm (rms = 1), eps inside the square root, rounded once to bf16;
 * what clarus_hip_rows_prologue would write for those rows. A tile covers whole rows.
 * No counterpart in the reference: it fuses its fused_gemm (kernels/gemm.py:353-400) with the
 * ln_rows pass of the next GEMM (kernels/spatial.py:312, ops/triton_cuda.py:104) for callers
 * that normalise a GEMM's output next (NAFNet conv3 -> conv4, conv5 -> conv1).
 */
int clarus_hip_gemm_ln_rows(const ClarusGemmArgs* args, void* ln_out, float eps, int32_t rms, void* stream);

/*
 * clarus_hip_gemm_ln_rows whose normalised rows feed a second GEMM in the same kernel instead
 * of being written: out2 = ln_rows . W2 + bias2 (K = 512, fp32 accumulation, rounded once to
 * bf16), with SimpleGate when gate2 = 1 (out2 channel c = (row c) * (row c + n2w / 2), dense
 * [m][n2w / 2]; else dense [m][n2w]). The same values clarus_hip_gemm_ln_rows followed by a
 * bf16 clarus_hip_gemm on ln_out (bias2, gate2) computes; args->c (the first GEMM's output) is
 * still written. n2w (W2's columns, the W^T rows) is a multiple of 512; bias2 fp32 [n2w] or
 * NULL. w2p holds W2^T [n2w][512] bf16 packed in MFMA fragment order: for pass P (512 W^T
 * rows), wave w (0..7), 16-k step s (0..31), block b (0..1), lane l (0..63): the 8 values
 * W^T[row(P, 64 w + 32 b + l % 32)][16 s + 8 (l / 32) + e], e = 0..7, where for r = 64 w + 32 b + i
 * with j = 16 ((i / 4) % 2) + 4 (i / 8) + i % 4: row(P, r) = 512 P + 64 w + 32 b + j, or with
 * gate2 = 1: b n2w / 2 + 256 P + 32 w + j (n2w * 512 bf16 in all).
 * No counterpart in the reference: it fuses fused_gemm (kernels/gemm.py:353-400), the ln_rows
 * pass (kernels/spatial.py:312) and the next fused_gemm, for callers that run a LayerNorm GEMM
 * right after a residual GEMM of width 512 (NAFNet conv3 -> conv4, conv5 -> conv1).
 */
int clarus_hip_gemm_ln_gemm(const ClarusGemmArgs* args, float eps, int32_t rms, const void* w2p, const float* bias2,
                            void* out2, int64_t n2w, int32_t gate2, void* stream);

/*
 * clarus_hip_gemm_ln_gemm for K = N = 512 and an fp32 residual, with the first GEMM's weight also
 * passed packed: w1p holds W1^T [512][512] in w2p's fragment order for one 512-row pass without
 * the gate (n2w = 512, gate2 = 0), and args->wt is not read. Both weights stream from L2 into
 * registers and the residual tile is staged in LDS during the first GEMM; args->c is written,
 * bit-identical to clarus_hip_gemm_ln_rows's output, and out2 as clarus_hip_gemm_ln_gemm's up
 * to the row statistics' summation order. args->pro may be CLARUS_PRO_MUL (bf16 A and map; small,
 * s_dtype, h, w, oh, ow, pt, pl as for clarus_hip_gemm, m a multiple of h w): the first GEMM's
 * A rows times the map, bit for bit clarus_hip_rows_prologue's rows, applied in the kernel.
 * No counterpart in the reference: the same fusion as clarus_hip_gemm_ln_gemm, for NAFNet's
 * level-3 pairs (conv3 -> conv4, conv5 -> conv1).
 */
int clarus_hip_gemm_ln_gemm_w1p(const ClarusGemmArgs* args, const void* w1p, float eps, int32_t rms, const void* w2p,
                                const float* bias2, void* out2, int64_t n2w, int32_t gate2, void* stream);

/*
 * Dense 3x3 convolution, stride 1, zero padding 1, as an implicit GEMM:
 *   y = act(conv3x3(up2 ? nearest_x2(x) : x) + bias) * out_scale (+ residual)
 * x [batch, h, w, cin] with pixel stride ldx (h, w = INPUT size); wt [cout][9 * cin] with
 * the reduction ordered (ky, kx, cin). Output [batch, H, W, cout] (H = 2h with up2) with
 * pixel stride ldo, or NCHW fp32 [batch, cout, H, W] with c_mode = CLARUS_C_NCHW (then the
 * residual is NCHW too). cin must be a multiple of 8.
 */
typedef struct ClarusConvArgs {
  const void* x;
  const void* wt;
  void* out;
  const float* bias; /* [cout] or NULL */
  const void* res;
  int64_t batch, h, w, cin, cout;
  int64_t ldx, ldo, ldr;
  int32_t x_dtype, w_dtype, o_dtype, r_dtype;
  int32_t act, up2, c_mode;
  float out_scale, slope;
  int32_t tile;
} ClarusConvArgs;

/* replaces kernels/conv3x3.py:123-168 conv3x3 (and the `ending` use of it) */
int clarus_hip_conv3x3(const ClarusConvArgs* args, void* stream);

/*
 * 3 -> cout 3x3 conv (padding 1) from an NCHW fp32 image [batch, 3, h, w] to NHWC
 * [batch, h, w, cout]; wt [27][cout] fp32 ordered (ky, kx, c); bias [cout] fp32. cout is a
 * multiple of 8, at most 512; out, wt and bias 16-byte aligned.
 * replaces kernels/conv3x3.py:196-204 intro3x3
 */
int clarus_hip_intro3x3(const float* inp, const float* wt, const float* bias, void* out,
                        int32_t out_dtype, int64_t batch, int64_t h, int64_t w, int64_t cout,
                        void* stream);

/*
 * Restormer MDTA attention map (python/clarus/ops/torch_ref.py:220-235):
 *   A[n, hd] = softmax((q / |q|) (k / |k|)^T * temperature[hd]) over c_h x c_h,
 * norms over all pixels. qkv [batch, h, w, 3c] contiguous (q | k | v channel blocks),
 * dtype qkv_dtype; out fp32 [batch, heads, c_h, c_h]; temperature fp32 [heads].
 * One launch: the pixel reduction is split over workgroups, whose partials are summed in the
 * same launch in a fixed order (deterministic). scratch must hold
 * clarus_hip_channel_attention_workspace(...) bytes; its first 64 KiB are arrival counters
 * that must be zero when a call starts, and every call leaves them zero (zero a new workspace
 * once, e.g. with a fill kernel, then reuse it call after call). Calls that overlap in time
 * must not share a workspace. At most 496 heads.
 * replaces kernels/attention.py:48-66 gram (gram_kernel :14-45) + ops/triton_cuda.py:174-181
 */
size_t clarus_hip_channel_attention_workspace(int64_t batch, int64_t hw, int64_t c, int64_t heads);
int clarus_hip_channel_attention(const void* qkv, int32_t qkv_dtype, const float* temperature,
                                 float* out, int64_t batch, int64_t hw, int64_t c,
                                 int64_t heads, void* scratch, size_t scratch_bytes,
                                 void* stream);

/*
 * clarus_hip_channel_attention without a workspace argument and without allocating: the split-K
 * partials live in a static device array of CLARUS_CHANNEL_ATTENTION_SCRATCH_MAX bytes, one per
 * device, held until the process ends (its address is looked up on the first call on each
 * device, with that device current). Its arrival counters are zero when the library loads and
 * every call leaves them zero. Same arguments, results and rules otherwise; shapes whose
 * clarus_hip_channel_attention_workspace(...) exceeds the maximum return CLARUS_EINVAL. Every
 * call on a device shares that device's array: calls that overlap in time on one device (other
 * streams, other threads) race and give wrong results. Calls no hipMalloc / hipFree.
 * No counterpart in the reference (its attention.py gram allocates its partials through torch);
 * for callers that cannot allocate device memory: code under HIP graph capture that must not
 * allocate, tight serving loops, harnesses that forbid allocation.
 */
#define CLARUS_CHANNEL_ATTENTION_SCRATCH_MAX (16u << 20)
int clarus_hip_channel_attention_noalloc(const void* qkv, int32_t qkv_dtype, const float* temperature,
                                         float* out, int64_t batch, int64_t hw, int64_t c,
                                         int64_t heads, void* stream);

/*
 * Per 8x8 patch and channel: y = irfft2(rfft2(patch) * g[c]) (+ residual), as the dense
 * real products  y = Inv[64 x 80] . (g_c * (Fwd[80 x 64] . x))  on fp32 MFMA.
 * fwd [80][64] and inv [64][80] fp32 (rows of re/im coefficients, see clarus_amd/dft.py);
 * gain [c][80] fp32 (the filter per coefficient). x [batch, h, w, c] NHWC with pixel
 * stride ldx; h, w multiples of 8 (the caller reflect-pads other sizes).
 * out [batch, h, w, c] contiguous, dtype o_dtype; residual contiguous like out or NULL.
 * replaces ops/torch_ref.py:253-270 patch_filter (torch-only in the reference)
 */
int clarus_hip_patch_filter(const void* x, int32_t x_dtype, int64_t ldx, const float* fwd,
                            const float* inv, const float* gain, const void* res,
                            int32_t r_dtype, void* out, int32_t o_dtype, int64_t batch,
                            int64_t h, int64_t w, int64_t c, void* stream);

/*
 * patch_filter(prologue(x) . W + bias) (+ residual) in one kernel: per 8x8 patch and output
 * channel, y = Inv . (g_c * (Fwd . z)) with z the patch's 64 values of the GEMM output, which
 * never leaves the registers. x [batch, h, w, k] contiguous (x_dtype); wt = W^T [n][k] (w_dtype,
 * bf16 or fp32); bias fp32 [n] or NULL; ln 0 = none, 1 = LayerNorm, 2 = RMS norm over the k
 * channels of each pixel (eps ln_eps, no affine; k <= 256; x and wt of one dtype), applied in
 * fp32; fwd / inv / gain as
 * clarus_hip_patch_filter with gain [n][80]. Sizes that are not multiples of 8 are reflect-padded
 * (h, w >= 9), which for a per-pixel GEMM is the GEMM of the reflected pixels. out [batch, h, w, n]
 * contiguous (o_dtype); residual contiguous like out or NULL. k % 8 == 0. With bf16 weights the
 * GEMM's A values enter bf16 MFMAs as hi + lo pairs where they are not bf16 already (2^-16
 * relative per operand); with fp32 weights it runs on fp32 MFMAs. The DFT products are those of
 * clarus_hip_patch_filter.
 * replaces kernels/freq.py:189-273 ln_gemm_patch_filter (ops/triton_cuda.py:260-272)
 */
int clarus_hip_linear_patch_filter(const void* x, int32_t x_dtype, const void* wt, int32_t w_dtype,
                                   const float* bias, int32_t ln, float ln_eps, const float* fwd,
                                   const float* inv, const float* gain, const void* res, int32_t r_dtype,
                                   void* out, int32_t o_dtype, int64_t batch, int64_t h, int64_t w,
                                   int64_t k, int64_t n, void* stream);

/*
 * FFTformer FSAS correlation (ops/torch_ref.py:278-288): per 8x8 patch,
 * irfft2(rfft2(q) * rfft2(k)) with q = x[..., :c], k = x[..., c:2c]; x has unit channel
 * stride and arbitrary batch / row / pixel strides (elements); out fp32 [batch, h, w, c].
 * fwd [80][64], inv [64][80] as above.
 * replaces kernels/freq.py:165-186 patch_corr
 */
int clarus_hip_patch_corr(const void* x, int32_t x_dtype, int64_t sn, int64_t sh, int64_t sw,
                          const float* fwd, const float* inv, float* out, int64_t batch,
                          int64_t h, int64_t w, int64_t c, void* stream);

/*
 * Depthwise 3x3 convolution, 'same' zero padding, dilation dil, fused gate (NHWC):
 *   y = conv_dw(x) + bias;  gate 0: out = act(y) (act CLARUS_ACT_NONE / CLARUS_ACT_GELU),
 *   gate 1: out = y[:, :c/2] * y[:, c/2:],  gate 2: out = gelu(y[:, :c/2]) * y[:, c/2:].
 * x [n, h, w, c] contiguous (x_dtype); w [9][c] fp32 taps (tap = 3 ky + kx); bias [c] fp32 or NULL;
 * out [n, h, w, c or c/2] contiguous (o_dtype). Output channels must be a multiple of 8.
 * Not a GEMM: the reference runs it on its torch backend (ops/torch_ref.py:143-155) or its
 * Triton dwconv (kernels/spatial.py:95-214); replaces the latter.
 */
int clarus_hip_dwconv3x3(const void* x, int32_t x_dtype, const float* w, const float* bias, void* out,
                         int32_t o_dtype, int64_t n, int64_t h, int64_t w_, int64_t c, int32_t dil,
                         int32_t gate, int32_t act, void* stream);

/*
 * TLC local mean (valid windows, NHWC): out[b, i, j, c] = mean of x[b, i .. i + k1 - 1,
 * j .. j + k2 - 1, c], i < h - k1 + 1, j < w - k2 + 1. x contiguous [n, h, w, c] (x_dtype),
 * out contiguous [n, h - k1 + 1, w - k2 + 1, c] (o_dtype); c a multiple of 8; scratch holds
 * clarus_hip_boxmean_workspace(...) bytes (the fp32 column sums). Sums are accumulated in fp64.
 * Not a GEMM: replaces the reference's boxmean (ops/torch_ref.py:133-141, ops/triton_cuda.py:132-137).
 */
size_t clarus_hip_boxmean_workspace(int64_t n, int64_t h, int64_t w, int64_t c, int64_t k1, int64_t k2);
int clarus_hip_boxmean(const void* x, int32_t x_dtype, void* out, int32_t o_dtype, int64_t n, int64_t h,
                       int64_t w, int64_t c, int64_t k1, int64_t k2, void* scratch, size_t scratch_bytes,
                       void* stream);

/*
 * PSNR and SSIM of two images on the device, basicsr's definitions (calculate_psnr /
 * calculate_ssim, crop_border 0): pred and gt contiguous uint8 [h, w, 3]; res[0] = PSNR in dB
 * (exact integer sum of squared differences; peak 1 when max(pred) <= 1, else 255; +inf for
 * identical images), res[1] = SSIM (the 11 x 11 x 11 Gaussian, sigma 1.5, over (h, w, channel)
 * with replicate padding, C1 = (0.01 peak)^2, C2 = (0.03 peak)^2, mean of the map; fp64
 * moments). res: 2 float64 on the device, written by the last kernel; no host synchronisation.
 * scratch holds clarus_hip_psnr_ssim_workspace(h, w) bytes, 16-byte aligned.
 * replaces python/clarus/metrics.py:59-159 (ssd_max_kernel, ssim_h_kernel, ssim_v_kernel) and
 * TritonMetrics.compute (:164-246)
 */
size_t clarus_hip_psnr_ssim_workspace(int64_t h, int64_t w);
int clarus_hip_psnr_ssim(const void* pred, const void* gt, int64_t h, int64_t w, double* res,
                         void* scratch, size_t scratch_bytes, void* stream);

/*
 * EVSSM's Mamba selective scan (one direction, no z gate, d_state 8) along each crop's raster
 * sequence: delta_l = softplus(dbl_l[0 .. r) . dt_w[d] + dt_b[d]);
 * h_l[n] = 2^(delta_l a2[d, n]) h_{l-1}[n] + delta_l dbl_l[r + n] u_l[d];
 * y_l[d] = sum_n dbl_l[r + 8 + n] h_l[n] + dsk[d] u_l[d], h_{-1} = 0.
 * u [t, l, d] contiguous (u_dtype bf16 or fp32); dbl [t, l, nc] fp32 (nc >= r + 16: dt_raw | B |
 * C); dt_w [d, r] (1 <= r <= 16), dt_b [d], a2 [d, 8] = A log2(e), dsk [d] fp32; y [t, l, d] fp32.
 * The sequence is cut into segments scanned in parallel and joined by their exact start states;
 * scratch holds clarus_hip_selective_scan_workspace(t, l, d) bytes. Deterministic.
 * replaces python/clarus/kernels/ssm.py:149-190 selective_scan (scan8_kernel, carry_kernel)
 */
size_t clarus_hip_selective_scan_workspace(int64_t t, int64_t l, int64_t d);
int clarus_hip_selective_scan(const void* u, int32_t u_dtype, const float* dbl, int64_t nc, const float* dt_w,
                              int64_t r, const float* dt_b, const float* a2, const float* dsk, float* y,
                              int64_t t, int64_t l, int64_t d, void* scratch, size_t scratch_bytes,
                              void* stream);

/* ABI version (CLARUS_HIP_ABI_VERSION) and struct sizes, for binding checks. */
int clarus_hip_abi_version(void);
size_t clarus_hip_sizeof_gemm_args(void);
size_t clarus_hip_sizeof_conv_args(void);

/* Text of the calling thread's last failure ("" if none). */
const char* clarus_hip_last_error(void);

/* Kernel chosen by the calling thread's last clarus_hip_gemm / clarus_hip_gemm_ln_rows /
   clarus_hip_gemm_ln_gemm / clarus_hip_conv3x3 call that launched ("" before any), e.g.
   "gemm_mfma32_kernel gate=0". A diagnostic, so that tests and benchmarks can record and
   compare which kernel served a problem; the dispatch never reads it. */
const char* clarus_hip_last_kernel(void);

#ifdef __cplusplus
}
#endif

#endif /* CLARUS_HIP_H */
