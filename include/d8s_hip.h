/* d8s_hip.h -- C ABI of libd8s_hip.so, the gfx950 kernels of the INT8 DenseNet encoder.
 *
 * The reference binds its CUDA kernels by name through ctypes (src/knee/cudart.py:87-152:
 * `Module.function`, `Function.launch` with by-value argument structs) and launches them from the
 * runner `Dense8SEncoder` (src/knee/dense8s.py:944-1488).  This library replaces that native
 * surface: every entry point below stands for one kernel family of the reference's final launch
 * sequence (src/knee/dense8s.py:1354-1385) and is called from Python through ctypes.
 *
 * Conventions (all entry points):
 *   - pointers are device pointers owned by the caller; nothing is allocated or freed here;
 *   - `stream` is a hipStream_t (PyTorch's `torch.cuda.Stream.cuda_stream`); every call is
 *     asynchronous on it and may be recorded into a HIP graph;
 *   - the return value is 0 on success, otherwise a hipError_t (invalid arguments give
 *     hipErrorInvalidValue = 1); the message of the last failure on the calling thread is
 *     d8s_last_error().
 *
 * Data layout (the reference's block "store", src/knee/dense8s_kernels.cu:10-14):
 *   in0  [N][G0][HW][32] int8   block input, 32 channels per group, channel c = 32 g + i;
 *   seg  [L][N][HW][32]  int8   layer outputs: layer l owns group G0 + l;
 *   bott [4][N*HW][32]   uint8  planar bottleneck: plane b holds channels 32 b .. 32 b + 31.
 * Channel c of pixel p holds x = sigma_c * q with q int8 (per-channel scale sigma).
 */
#ifndef D8S_HIP_H
#define D8S_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define D8S_ABI_VERSION 1

/* Arguments of the 1x1 GEMMs (conv1 and the transition).  Same fields and meaning as the
 * reference's `struct KArg` (src/knee/dense8s_kernels.cu:146-158, src/knee/dense8s.py:76-82),
 * plus `wsum`: gfx950's int8 MFMA multiplies signed bytes, so the unsigned prologue output u is fed
 * as u - 128 and the GEMM adds 128 * sum_k w[o][k] back (exact in int32).
 *   in0, seg  the block store (see above);  G0 groups in in0, G groups read (G0 + layers so far);
 *   w         weights [G][cout][32] int8 (the reference's `_chunked`, dense8s.py:436-440);
 *   abh       fp16 prologue table [G*16][4] = (A_2p, A_2p+1, B_2p, B_2p+1) (dense8s.py:443-449);
 *   gd        epilogue table [cout][2] float: conv1 (g, d) of `L*_gdu`; transition (k', 0) of
 *             `T*_gdf` (dense8s.py:485-486,500-501);
 *   wsum      [cout] int32, sum over k of w[o][k];
 *   out       conv1: planar u8 bottleneck [4][rows][32]; transition: next block's in0
 *             [N][G0n][HW/4][32];
 *   N, HW, W  images, pixels per image, image width;  rows = N*HW;  cout output channels. */
typedef struct D8sGemmArgs {
    const int8_t* in0;
    const int8_t* seg;
    const int8_t* w;
    const uint16_t* abh;
    const float* gd;
    const int32_t* wsum;
    void* out;
    int32_t G0, G, N, HW, W, rows, cout, G0n;
} D8sGemmArgs;

/* Arguments of the 3x3 conv (pad 1, 128 -> 32).  Same meaning as the reference's `struct C2Arg`
 * (src/knee/dense8s_kernels.cu:1936-1942, src/knee/dense8s.py:131-137) without the rectangle fields,
 * which this library chooses itself, plus `wsum` (see D8sGemmArgs).
 *   x     planar u8 bottleneck [4][N*H*W][32];
 *   w     weights [4][9][32][32] int8 = [input block][tap][output][input] (`L*_w2k`, dense8s.py:487-488);
 *   sc    [32] float requantisation scale c2u (dense8s.py:489);
 *   wsum  [32] int32, sum over (input channel, tap) of w;
 *   out   the layer's store slot [N][H*W][32] int8. */
typedef struct D8sConv2Args {
    const uint8_t* x;
    const int8_t* w;
    const float* sc;
    const int32_t* wsum;
    int8_t* out;
    int32_t N, H, W, pad_;
} D8sConv2Args;

/* Arguments of a whole dense layer, conv1 and conv2 fused (d8s_dense): the fields of D8sGemmArgs for
 * conv1 and of D8sConv2Args for conv2, the bottleneck staying on chip.  Same role as the reference's
 * `struct TileArg` + `struct LayerP` of its fused "tile" layer (src/knee/dense8s_kernels.cu:996-1003,
 * 1441-1447; src/knee/dense8s.py:139-152).
 *   in0, seg, G0, G   the block store and the groups read (as D8sGemmArgs);
 *   w1, abh, gd, w1sum  conv1 weights [G][128][32], prologue table, epilogue table [128][2] (g, d),
 *                     sum_k w1[o][k] [128];
 *   w2, sc, w2sum     conv2 weights [4][9][32][32], requantisation scale [32], weight sums [32];
 *   out               the layer's store slot [N][H*W][32];  N, H, W images and their size. */
typedef struct D8sDenseArgs {
    const int8_t* in0;
    const int8_t* seg;
    const int8_t* w1;
    const uint16_t* abh;
    const float* gd;
    const int32_t* w1sum;
    const int8_t* w2;
    const float* sc;
    const int32_t* w2sum;
    int8_t* out;
    int32_t G0, G, N, H, W, pad_;
} D8sDenseArgs;

/* The tables of one dense layer for d8s_dense_block (fields as in D8sDenseArgs).  The reference's
 * `struct LayerP` (src/knee/dense8s_kernels.cu:996-1003) plus the weight sums. */
typedef struct D8sLayerP {
    const int8_t* w1;
    const uint16_t* abh;
    const float* gd;
    const int32_t* w1sum;
    const int8_t* w2;
    const float* sc;
    const int32_t* w2sum;
} D8sLayerP;

/* Arguments of a whole dense block (d8s_dense_block): the block store (in0 [N][G0][H*W][32], seg
 * [L][N][H*W][32]), `layers` a DEVICE array of L D8sLayerP (layer l reads G0 + l groups and writes
 * slot l).  The reference's `struct ImgArg` (src/knee/dense8s_kernels.cu:1005-1011,
 * src/knee/dense8s.py:155-159). */
typedef struct D8sBlockArgs {
    const int8_t* in0;
    int8_t* seg;
    const D8sLayerP* layers;
    int32_t N, H, W, G0, L, pad_;
} D8sBlockArgs;

/* Arguments of a whole dense block with every image split into `parts` row bands (d8s_dense_block_parts):
 * the block store and layer tables as D8sBlockArgs, plus the caller's synchronisation memory.
 *   sync   device, D8S_PARTS_SYNC_WORDS(N * parts) uint32, all zero before the first call.  Words 0-1
 *          (ticket and end count) are zero again after every call, word 2 counts bounded waits that
 *          ran out (0 when the results are valid; only the caller clears it), word 3 counts the
 *          launches (it names each launch's exchange rows);
 *   xchg   device, D8S_PARTS_XCHG_BYTES(N * parts, W) bytes, all zero before the first call: the
 *          bottleneck rows a part hands to its neighbours, as (value, tag) pairs;
 *   parts  row bands per image: H % parts == 0, (H / parts) * W in {32, 64, 128, 256}, parts at most
 *          the device's compute units (d8s_parts_supported(H, W, G0 + L - 1, parts) says whether a
 *          shape is taken).
 * One runner's buffers serve its calls in stream order; two launches in flight at once need their own.
 * Forward progress: a workgroup takes the next (image, band) ticket when it starts, so the running
 * workgroups of a launch always hold a prefix of its tickets, and every image wholly inside that prefix
 * completes without waiting for anything else.  The waits therefore end whenever the launches in flight
 * on the device together have no more bands per image than it has compute units: a wait can only run
 * out (word 2) when other work keeps CUs busy for about a second.  Callers that must never use such
 * results pass word 2 to d8s_final_checked, which then writes NaN features. */
#define D8S_PARTS_SYNC_WORDS(nparts) (64 + 0 * (nparts))
#define D8S_PARTS_XCHG_BYTES(nparts, W) ((uint64_t)(nparts) * 1024 * (W))
typedef struct D8sPartsArgs {
    const int8_t* in0;
    int8_t* seg;
    const D8sLayerP* layers;
    uint32_t* sync;
    uint8_t* xchg;
    int32_t N, H, W, G0, L, parts;
} D8sPartsArgs;

/* Arguments of the stem: 7x7/2 conv (pad 3) with norm0 folded in, bias, ReLU, 3x3/2 max-pool (pad 1)
 * and per-channel int8 quantisation into the first block's in0.  Replaces the reference's TensorRT
 * fp16 stem engine + `quant_seg` (src/knee/dense8s.py:684-716,1330-1352;
 * src/knee/dense8s_kernels.cu:2365-2412), with the uint8 normalisation and flip of the input fused
 * into the load (the role of `gather_u8_to_f16`, src/knee/data/fused_uint8.py:480-506).
 *   x      input [N][3][H][W]: uint8 when kind = D8S_IN_U8 (x16 = lut[c][u]; 4-byte aligned), fp16
 *          when kind = D8S_IN_F16 (used as is; 8-byte aligned when W <= 512);
 *   lut    [3][256] fp16 (kind = D8S_IN_U8 only);
 *   w16    [64][168] fp16, norm0 folded in, k = (channel * 7 + ky) * 8 + kx + 1 and k % 8 = 0
 *          zero: the reference's `S_w16` table (src/knee/dense8s.py:522-530);
 *   bias   [64] float;  inv [64] float = 1 / sigma0;
 *   out    in0 of block 0 [N][2][(H/4)*(W/4)][32];
 *   flip   0: as is; 1: every image mirrored horizontally (x[..., W-1-j]); 2: flip-TTA pairs, N even:
 *          x holds N/2 images, output image n < N/2 is image n, output image n >= N/2 is image
 *          n - N/2 mirrored. */
#define D8S_IN_F16 0
#define D8S_IN_U8 1
typedef struct D8sStemArgs {
    const void* x;
    const uint16_t* lut;
    const uint16_t* w16;
    const float* bias;
    const float* inv;
    int8_t* out;
    int32_t N, H, W, kind, flip, pad_;
} D8sStemArgs;

/* conv1 of a dense layer: u = RNE(255 sat(fp16(A q + B))) per input channel (prologue), acc = sum_k
 * w[o][k] u[k] (int32, i8 MFMA), v = low byte of fma(sat(fma(g, acc, d)), 255, 2^23) into the planar
 * bottleneck.  cout must be 128.  Replaces `conv1_w64_pl` (src/knee/dense8s_kernels.cu:479-627,
 * launch src/knee/dense8s.py:1205-1240). */
int d8s_conv1(const D8sGemmArgs* a, void* stream);

/* The same GEMM writing the int32 accumulators acc[rows][cout] (and the bottleneck too when
 * a->out is not NULL).  The reference has no such kernel: its checks recompute the accumulators
 * (kaggle/int8_pack/pack_dense8s.py:246-283); here they are compared bit for bit. */
int d8s_conv1_acc32(const D8sGemmArgs* a, int32_t* acc, void* stream);

/* Kernel variants of conv1, conv2 and the transition, for tuning on the device: the same bytes from a
 * chosen kernel.  The role of the reference's `tune_bm` / `tune_c2` / `tune_trans`
 * (src/knee/dense8s.py:1598-1651), whose packages record a kernel per layer and block
 * (kaggle/int8_pack/pack_dense8s.py:141-147).  d8s_*_variant(a, v) returns the variant that a launch
 * with v runs: v itself, or for v = 0 the choice of d8s_conv1 / d8s_conv2 / d8s_transition; -1 where
 * the arguments or the shape do not take v.  d8s_*_as(a, v, stream) launches it (an error where it
 * is not taken).
 *   conv1       1 persistent, 32-pixel tiles; 2 persistent, 64-pixel tiles (both: rows < 2^34, in0
 *               and a slot below 4 GiB); 3, 4, 5 one pass with 1, 2, 4 k-slices.
 *   conv2       tile TW x TH: 1 32x8, 2 32x4, 3 32x2, 4 16x4, 5 8x8, 6 4x16, 7 2x32, 8 1x64 (from 3
 *               on the K steps split over 4 waves), for maps at least TW wide.
 *   transition  activation prefetch depth / weight sets: 1 4/2 (G a multiple of 4), 2 4/4 (G a
 *               multiple of 4, cout in 416..640), 3 2/2 (G even), 4 1/1. */
int d8s_conv1_variant(const D8sGemmArgs* a, int32_t variant);
int d8s_conv1_as(const D8sGemmArgs* a, int32_t variant, void* stream);
int d8s_conv2_variant(const D8sConv2Args* a, int32_t variant);
int d8s_conv2_as(const D8sConv2Args* a, int32_t variant, void* stream);
int d8s_transition_variant(const D8sGemmArgs* a, int32_t variant);
int d8s_transition_as(const D8sGemmArgs* a, int32_t variant, void* stream);

/* conv2 of a dense layer: acc = sum over taps and input channels (zero padding) of w u (int32,
 * i8 MFMA), q = RNE(clamp(float(acc) * sc[o], -127, 127)) into the store slot.  Replaces
 * `conv2_t8x32_pl` / `conv2_t16x16_pl` (src/knee/dense8s_kernels.cu:2679-2832, launch
 * src/knee/dense8s.py:1274-1290). */
int d8s_conv2(const D8sConv2Args* a, void* stream);

/* A dense layer in one launch: conv1 as d8s_conv1 into a bottleneck that stays in LDS, then conv2 as
 * d8s_conv2 into the layer's store slot; the bytes written equal those of d8s_conv1 + d8s_conv2 (the
 * same integer sums and epilogues).  The spatial tile's halo is recomputed: no bottleneck in HBM.
 * Replaces the reference's fused layer `dense_tile7` (src/knee/dense8s_kernels.cu:1449-1699, launch
 * src/knee/dense8s.py:1154-1203, kind "tile"). */
int d8s_dense(const D8sDenseArgs* a, void* stream);

/* conv2 of layer l, then conv1 of layer l + 1, in one launch: c2 as for d8s_conv2 (x = layer l's
 * bottleneck, out = layer l's store slot), c1 as for d8s_conv1 (G = G0 + l + 1 groups, the last of
 * which is c2's output slot; out = layer l + 1's bottleneck, a buffer other than c2->x).  The bytes
 * written equal those of d8s_conv2(c2) followed by d8s_conv1(c1): the new 32 channels reach conv1 from
 * registers, so a block of L layers runs in L + 1 launches (conv1 of layer 0, L - 1 of these, conv2 of
 * layer L - 1) instead of 2 L.  Maps W = 16, 32 or 64 wide with H * W a multiple of 128 and
 * 2 <= G <= D8S_C21_MAX_GROUPS (d8s_c21_supported(H, W, G) says whether a shape is taken).  Replaces
 * the pair of launches conv2 (layer l), conv1 (layer l + 1) of the reference's per-layer sequence
 * (src/knee/dense8s.py:1354-1385; kernels `conv2_t8x32_pl` and `conv1_w64_pl`,
 * src/knee/dense8s_kernels.cu:2679-2832, 479-627). */
#define D8S_C21_MAX_GROUPS 64
int d8s_conv2_conv1(const D8sConv2Args* c2, const D8sGemmArgs* c1, void* stream);
int d8s_c21_supported(int32_t H, int32_t W, int32_t G);

/* Every layer of a dense block in one launch, one workgroup per image, for maps of at most 256
 * pixels with G0 + L - 1 <= 64: the bytes of d8s_conv1 + d8s_conv2 layer after layer.  Replaces the
 * reference's whole-block fused kernels `dense_img*` (src/knee/dense8s_kernels.cu:1005-1219, launch
 * src/knee/dense8s.py:1154-1203). */
int d8s_dense_block(const D8sBlockArgs* a, void* stream);

/* Every layer of a dense block in one launch with each image split into row bands (see D8sPartsArgs), one
 * workgroup per band: the bytes of d8s_conv1 + d8s_conv2 layer after layer, with N * parts workgroups
 * instead of N, for batches too small to fill the chip with one workgroup per image.  Neighbouring
 * bands hand each other their boundary bottleneck rows once per layer through `xchg`.  The whole-block
 * role of the reference's `dense_img*` kernels (src/knee/dense8s_kernels.cu:1005-1219), which run
 * one image per block. */
int d8s_dense_block_parts(const D8sPartsArgs* a, void* stream);
int d8s_parts_supported(int32_t H, int32_t W, int32_t G, int32_t parts);

/* Transition: prologue on the 4 pixels of every 2x2 square, s = sum of the four u, S = sum_k w[o][k]
 * s[k] (exact int32), q = RNE(clamp(k'_o * (float(S) / 4), -127, 127)) into the next block's in0.
 * H and W even, cout a multiple of 32 (at most 1024), N * HW < 2^31 and the in0 / one seg slot below
 * 4 GiB.  Replaces `trans_w0` / `trans_w1`
 * (src/knee/dense8s_kernels.cu:3041-3262, launch src/knee/dense8s.py:1242-1272). */
int d8s_transition(const D8sGemmArgs* a, void* stream);

/* Final features: out[n][c] = (sum over the four strided partials of sum_p relu(fma(a_c, q, b_c))) / HW,
 * norm5 with sigma folded in (ab = `F_ab` [ctot][2]).  Replaces `final_q`
 * (src/knee/dense8s_kernels.cu:2304-2323, launch src/knee/dense8s.py:1380-1384); same arguments. */
int d8s_final(const int8_t* in0, int32_t G0, const int8_t* seg, int32_t N, int32_t HW,
              const float* ab, float* out, int32_t ctot, void* stream);

/* d8s_final for a pass with banded whole-block launches (d8s_dense_block_parts): `status` is the
 * device word those launches count expired waits in (D8sPartsArgs.sync + 2).  When it is not zero,
 * every feature of the pass is NaN instead of values computed from stale halo rows.  `report` (may
 * be NULL) is a host-mapped word (d8s_host_mapped) that receives the status word, so that the host
 * can see an error after the pass without a synchronisation.  No counterpart in the reference, whose
 * whole-block kernel runs one workgroup per image and never waits on another (the role of its
 * `final_q`, src/knee/dense8s_kernels.cu:2304-2323). */
int d8s_final_checked(const int8_t* in0, int32_t G0, const int8_t* seg, int32_t N, int32_t HW,
                      const float* ab, float* out, int32_t ctot, const uint32_t* status, uint32_t* report,
                      void* stream);

/* The device address of pinned host memory (hipHostGetDevicePointer), for d8s_final_checked's
 * `report`.  Plumbing without a reference counterpart (the reference reads its results with copies). */
int d8s_host_mapped(void* host, void** dev);

/* Linear head on the final features: out[n][k] = b[k] + sum_c x[n][c] w[k][c] in float32 (x [N][C],
 * w [K][C], b [K], out [N][K]; K <= 4096).  Configuration 4's 1664 -> 8 logits after the encoder; the
 * reference runs its head right after the encoder on the same device (src/knee/infer.py:1015-1017). */
int d8s_linear(const float* x, int32_t N, int32_t C, const float* w, const float* b, int32_t K, float* out,
               void* stream);

/* Stem (see D8sStemArgs).  H and W multiples of 4.  Widths up to 512 run a row-band kernel (pooling
 * in registers, one quantisation per pooled value), wider ones a tile kernel; both give the same bytes. */
int d8s_stem(const D8sStemArgs* a, void* stream);

/* Paired launches.  No counterpart in the reference: for callers running two encoders of the same
 * geometry over the same batch shape (the final model's two weight seeds), each of these runs the
 * same step for both in ONE launch -- the same work and bytes as the two single calls, but a 96-image
 * pass's small late layers then fill the chip between them instead of one pass at a time (the 16 x 16
 * whole block: 96 workgroups per pass, 192 for the pair in the time of one).  `a` and `b` must agree
 * in every shape field (N, H, W, group counts, cout, input kind and flip); their buffers and tables
 * are independent and must not overlap.  Kernel forms without a pair launch (split-K conv1, the 2-D
 * fused tile, the wide-image stem) run as two launches. */
int d8s_stem_pair(const D8sStemArgs* a, const D8sStemArgs* b, void* stream);
int d8s_conv1_pair(const D8sGemmArgs* a, const D8sGemmArgs* b, void* stream);
int d8s_conv2_pair(const D8sConv2Args* a, const D8sConv2Args* b, void* stream);
int d8s_dense_pair(const D8sDenseArgs* a, const D8sDenseArgs* b, void* stream);
int d8s_dense_block_pair(const D8sBlockArgs* a, const D8sBlockArgs* b, void* stream);
int d8s_transition_pair(const D8sGemmArgs* a, const D8sGemmArgs* b, void* stream);

/* ---- Upstream preprocessing: raw uint16 crops -> resize -> exact 1/99 percentiles -> uint8 ----------
 *
 * The reference turns the raw crop of every series into the uint8 stacks the encoder reads on the GPU
 * (src/knee/data/raw_crop.py:492-549 `payloads_to_uint8_torch`): per stack (one series at one crop
 * scale) the stored uint16 values, Rescale `u * slope + intercept` in float32 (raw_crop.py:520-522),
 * the crop box, the resize to img x img of `_resize_torch` (raw_crop.py:419-432: cv2 INTER_AREA
 * tables when the box is taller than img, torch bilinear with align_corners=False otherwise, the
 * values themselves at img x img), then the linear np.percentile at (1, 99) selected exactly, float64
 * `(x - lo) * (255 / (hi - lo))` clipped to [0, 255] and truncated (`cache._to_uint8`,
 * src/knee/data/cache.py:319-340, on the GPU `to_uint8_torch_hist_batch`, torch_uint8.py:332-357, and
 * the NVRTC `hist_to_uint8`, fused_uint8.py:847-872), a stack whose percentiles are not finite or
 * equal (or that holds a NaN) being all zero, and the side flip (raw_crop.py:541-545).
 *
 * d8s_prep runs all of it for up to D8S_PREP_MAX_STACKS stacks in one call: the resize runs once,
 * into the caller's scratch buffer, together with the first histogram pass; the later passes read the
 * float32 stacks.  kind 1 starts from float32 stacks already at img x img instead
 * (`to_uint8_torch_hist_batch(x)`; box, resc and scratch ignored).
 * The uint8 values are bit-identical to `cache._to_uint8` of the resized stack. */
#define D8S_PREP_MAX_STACKS 16
#define D8S_PREP_MAX_TAPS 16
#define D8S_FLIP_NONE 0
#define D8S_FLIP_X 1          /* columns reversed (Coronal / Axial of a right knee) */
#define D8S_FLIP_SLICES 2     /* slices reversed (Sagittal of a right knee) */

/* One stack.  r1/g1 and r2/g2: the percentiles are lerp(sorted[r], sorted[r + 1], g) over the
 * n = (k1 - k0) * img * img values, numpy's linear method (torch_uint8.py:31-42 `_ranks`). */
typedef struct D8sPrepStack {
    uint64_t src;       /* kind 0: uint16 region [K][hr][wr]; kind 1: float32 [K][img][img] (16-byte aligned) */
    uint64_t resc;      /* kind 0: float32 [K][2] slope and intercept per slice, or 0 for none */
    uint64_t out;       /* d8s_prep: uint8 [K][img][img] (8-byte aligned);
                         * d8s_prep_resize: float32 [K][img][img] (16-byte aligned) */
    int32_t K, hr, wr;  /* slices of the stack; region rows and columns (kind 0) */
    int32_t y0, y1, x0, x1;  /* crop box in the region (kind 0) */
    int32_t k0, k1;     /* slices [k0, k1) are computed (`read_range`, raw_crop.py:79-90); the output
                         * slices outside the range are not written */
    int32_t flip;       /* D8S_FLIP_*: applied to the uint8 output of d8s_prep */
    int32_t r1, r2;     /* lower order statistics of the 1st and 99th percentile */
    double g1, g2;      /* their gamma */
} D8sPrepStack;

/* What d8s_prep leaves at the start of the workspace for stack i: the percentiles (float64), the
 * scale 255 / (hi - lo) and whether the stack was written as zeros. */
typedef struct D8sPrepStat {
    double lo, hi, scale;
    int32_t bad, pad_;
} D8sPrepStat;

typedef struct D8sPrepArgs {
    uint64_t workspace;   /* device memory, 256-byte aligned, d8s_prep_workspace bytes; starts with
                           * D8sPrepStat[D8S_PREP_MAX_STACKS] */
    uint64_t ws_bytes;
    uint64_t scratch;     /* d8s_prep, kind 0: device memory, 16-byte aligned, of at least
                           * 4 * sum over the stacks of (k1 - k0) * img * img bytes: the resized float32
                           * stacks (written once, read by the later passes); otherwise unused */
    uint64_t scratch_bytes;
    int32_t kind;         /* 0: uint16 regions; 1: float32 stacks at img x img */
    int32_t img;          /* output side, a multiple of 8, 8 .. 4096 */
    int32_t n_stacks;     /* 1 .. D8S_PREP_MAX_STACKS */
    int32_t pad_;
    D8sPrepStack s[D8S_PREP_MAX_STACKS];
} D8sPrepArgs;

/* Bytes of workspace d8s_prep and d8s_prep_resize need for n_stacks stacks of side img. */
int d8s_prep_workspace(int32_t n_stacks, int32_t img, uint64_t* bytes);

/* Resize + percentiles + uint8 + flip of every stack (see above).  Ranks: 0 <= r1, r1 + 1 < n,
 * r2 + 1 < n, n >= 4; area tables (box taller than img) of at most D8S_PREP_MAX_TAPS taps per axis. */
int d8s_prep(const D8sPrepArgs* a, void* stream);

/* kind 0 only: the resized float32 stacks themselves (`_resize_torch` after the Rescale,
 * raw_crop.py:419-432,520-527) into `out`, slices [k0, k1); flip and ranks are ignored. */
int d8s_prep_resize(const D8sPrepArgs* a, void* stream);

/* ---- Geometric TTA view: bilinear grid sampling of fp16 windows --------------------------------
 *
 * The reference's zoom / shift view (src/knee/tta.py:131-148 `affine_windows`: `F.affine_grid` once,
 * expanded, then `F.grid_sample(mode="bilinear", padding_mode="zeros", align_corners=False)` in fp16)
 * applied to windows gathered from the uint8 volume (src/knee/infer.py:973-1012: `gather_u8_f16`,
 * src/knee/data/fused_uint8.py:480-506, then `affine_windows`).  One grid [H][W][2] (fp16, the output
 * of `F.affine_grid`) is shared by every image.
 *   kind 0: src fp16 images [N][H][W] (N = windows x depth), out[n] = sample(src[n]);
 *   kind 1: src uint8 volume [B][SK][H][W], slice_idx int64 [M], lut fp16 [256] (u / 255):
 *           out[b * M + m] = sample(lut[src[b][slice_idx[m]]]), N = B * M (the fused gather); with
 *           grid = 0 the gather alone, out = lut[...] (the identity view).  slice_idx is read on the
 *           device and not checked (a check would synchronise): an index outside 0 .. SK-1 is clamped
 *           into it (reads stay inside the volume); callers validate the indices once.
 * Arithmetic: that of torch's grid_sampler_2d kernel in float32 (source index
 * fma(g + 1, size, -1) / 2, weights (x_se - x)(y_se - y) ..., taps accumulated by fma in the order
 * nw, ne, sw, se, out of range taps skipped), rounded once to fp16. */
typedef struct D8sGridArgs {
    uint64_t src;        /* see kind */
    uint64_t slice_idx;  /* kind 1 */
    uint64_t lut;        /* kind 1 */
    uint64_t grid;       /* fp16 [H][W][2] (kind 1: 0 for the gather alone) */
    uint64_t out;        /* fp16 [N][H][W] */
    int32_t kind, N, H, W;
    int32_t B, SK, M, pad_;  /* kind 1 */
} D8sGridArgs;

int d8s_grid_sample(const D8sGridArgs* a, void* stream);

/* ---- The head after the encoder --------------------------------------------------------------
 *
 * The final model's `KneeBaseline` head on the encoder's window features (src/knee/models/
 * baseline.py: `_features_full` :870-932, `_context` :954-977, `forward` :1083-1170; configuration
 * configs/exp/376-full-data-v9j-287-img512.yaml: one context layer of width 256, 4 heads, attention
 * pooling), for B studies of W windows, in float32:
 *   f   = z + slot_emb[slot_of[w]]                                   (B, W, D)
 *   h   = ctx_in(f) + ctx_pos[w % PER]; one pre-norm transformer encoder layer on h (self-attention,
 *         keys of absent slots masked, all keys when no slot is present; ReLU feed-forward of FF);
 *   f2  = f + ctx_out(h)
 *   a   = attn(f2) (B, W, T), -inf on absent slots (0 everywhere if none is present), softmax over W
 *   logits[b][t] = sum_w a (f2 . cls_w[t]) + cls_b[t]                 (B, T)
 * Weights in torch's Linear layout [out][in]; the transformer layer's are those of
 * `nn.TransformerEncoderLayer` (self_attn.in_proj, self_attn.out_proj, linear1, linear2, norm1, norm2).
 * W <= 128, CD = 64 x heads, T <= 16.  slot_mask [B][S] uint8; the reference's window_index is not
 * used by this configuration (context_pos None: the position is w % PER).  slot_of is read on the
 * device and not checked (a check would synchronise): an entry outside 0 .. S-1 reads no memory, its
 * windows take no slot embedding and count as absent, where the reference raises; callers validate
 * the map once. */
typedef struct D8sHeadArgs {
    const float* z;            /* [B][W][D] encoder features */
    const int32_t* slot_of;    /* [W] */
    const uint8_t* slot_mask;  /* [B][S] */
    const float* slot_emb;     /* [S][D] */
    const float *ctx_in_w, *ctx_in_b, *ctx_pos;            /* [CD][D], [CD], [PER][CD] */
    const float *in_proj_w, *in_proj_b, *out_proj_w, *out_proj_b;  /* [3CD][CD], [3CD], [CD][CD], [CD] */
    const float *ln1_w, *ln1_b, *ln2_w, *ln2_b;            /* [CD] */
    const float *ff1_w, *ff1_b, *ff2_w, *ff2_b;            /* [FF][CD], [FF], [CD][FF], [CD] */
    const float *ctx_out_w, *ctx_out_b;                    /* [D][CD], [D] */
    const float *attn_w, *attn_b, *cls_w, *cls_b;          /* [T][D], [T], [T][D], [T] */
    float* logits;             /* [B][T] */
    void* workspace;           /* device memory of d8s_head_workspace bytes, 256-byte aligned */
    uint64_t ws_bytes;
    int32_t B, W, D, S, CD, heads, FF, PER, T, ctx_layers;   /* ctx_layers must be 1 */
} D8sHeadArgs;

int d8s_head_workspace(const D8sHeadArgs* a, uint64_t* bytes);
int d8s_head(const D8sHeadArgs* a, void* stream);

/* d8s_head without a workspace argument and without any allocation: no counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as d8s_head; a->workspace and
 * a->ws_bytes are ignored.  The workspace is a static device array of D8S_HEAD_SCRATCH_BYTES per GPU
 * (32 MiB: up to 16 studies of 128 windows, or 23 of 88, at the final configuration), held until the
 * process ends; a call whose d8s_head_workspace() exceeds it is rejected with hipErrorInvalidValue.
 * `stream` must belong to the current device.  Every call on a GPU uses that GPU's one array, so calls
 * that overlap on one GPU (unordered streams) race: order them on one stream or with events. */
#define D8S_HEAD_SCRATCH_BYTES (32u << 20)
int d8s_head_noalloc(const D8sHeadArgs* a, void* stream);

/* Library identification: "d8s-hip <abi> <source hash> gfx950". */
const char* d8s_version(void);

/* Message of the last failed call on the calling thread ("" if none). */
const char* d8s_last_error(void);

/* Diagnostics (the reference's micro-benchmarks, src/knee/dense8s_kernels.cu:4232-4417).
 * d8s_micro_copy: dst[i] = src[i] over `bytes` (a multiple of 16): the HBM bandwidth floor.
 * d8s_micro_mfma: `blocks` workgroups each running `iters` rounds of independent
 *   v_mfma_i32_32x32x32_i8 on 4 waves; sink receives one value per block (keeps the work alive).
 * d8s_probe_mfma_i8: D = A B for one 32x32x32 int8 MFMA tile, A [32][32] and B [32][32]
 *   row-major (B indexed [k][j]), D [32][32] int32 row-major: checks this library's operand and
 *   result lane layout.
 * d8s_probe_mfma_f16: the same for one 32x32x16 fp16 MFMA tile, A [32][16], B [16][32] fp16 bits,
 *   D [32][32] float. */
int d8s_micro_copy(const void* src, void* dst, size_t bytes, void* stream);
int d8s_micro_mfma(int32_t blocks, int32_t iters, int32_t* sink, void* stream);
int d8s_probe_mfma_i8(const int8_t* A, const int8_t* B, int32_t* D, void* stream);
int d8s_probe_mfma_f16(const uint16_t* A, const uint16_t* B, float* D, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* D8S_HIP_H */
