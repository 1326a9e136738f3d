// gfx950 kernels of the head that follows the encoder (the reference's `KneeBaseline` context and
// per-finding attention pooling, src/knee/models/baseline.py:870-932,954-977,1083-1170) and their C
// ABI, d8s_head (include/d8s_hip.h).
//
// Per study (W windows of D-dim encoder features, a few hundred KB) the head is a few small matrix
// products with row-wise normalisations around them; the PyTorch head is ~30 launches of tiny
// kernels.  Here it is 10 to 15 launches (with the split-K sums) for all studies of a call, float32 throughout:
//   1. k_head_gemm<PRO_SLOT, EPI_BIAS_POS>: h = (z + slot_emb[slot]) ctx_in^T + b + ctx_pos[w % per]
//   2. k_head_gemm<PRO_LN, EPI_BIAS>:       qkv = LN1(h) in_proj^T + b
//   3. k_head_attn:                          per (study, head, 16 queries) softmax(q k^T / sqrt(dh), keys of
//                                            absent slots masked) v
//   4. k_head_gemm<PRO_NONE, EPI_BIAS_RES>:  h1 = h + att out_proj^T + b
//   5. k_head_gemm<PRO_LN, EPI_BIAS_RELU>:   u = relu(LN2(h1) ff1^T + b)
//   6. k_head_gemm<PRO_NONE, EPI_BIAS_RES>:  h2 = h1 + u ff2^T + b
//   7. k_head_gemm<PRO_NONE, EPI_DOTS>:      f2 = z + slot_emb + h2 ctx_out^T + b, and per 64-column
//                                            block the partial dots of f2 with attn.weight and cls_w
//   8. k_head_dotsum:                        the partial dots summed over the column blocks
//   9. k_head_pool:                          per study: a = attn(f2) masked, softmax over windows,
//                                            logits = sum_w a (f2 . cls_w) + cls_b
// (one context layer: the final model's configuration.)  A product whose 64 x 64 tiles are too few
// to fill the chip (the 1664-deep ctx_in above all) is split over K into workgroups that write raw
// sums, added in split order with the epilogue by k_head_splitk.  The pooled vector of the reference,
// sum_w a f2, is never formed: its dot with cls_w is sum_w a (f2 . cls_w), the same value up to the
// order of the float32 sums.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "d8s_hip.h"
#include "d8s_host.h"

#define DEV __device__ __forceinline__
#define INLINE_H __attribute__((always_inline))

namespace {

constexpr int NT = 256;
constexpr int TM = 64, TN = 64, KC = 64;     // product tile: 64 rows x 64 columns, K in chunks of 64
constexpr int WMAX = 128;                    // windows per study
constexpr int TMAX = 16;                     // findings

enum Pro { PRO_NONE = 0, PRO_SLOT = 1, PRO_LN = 2 };
enum Epi { EPI_BIAS = 0, EPI_BIAS_POS = 1, EPI_BIAS_RES = 2, EPI_BIAS_RELU = 3, EPI_DOTS = 4 };

struct GemmP {
    const float* A;      // [M][K] (lda = K)
    const float* Bw;     // [N][K] weights (torch Linear layout)
    const float* bias;   // [N]
    float* C;            // [M][ldc]
    int M, N, K, ldc;
    // PRO_SLOT: A row r gets + slot_emb[slot_of[r % W]] (nothing for a slot outside 0 .. S-1)
    const float* slot_emb;
    const int32_t* slot_of;
    int W, S;
    // PRO_LN: A row normalised with ln_w, ln_b (eps 1e-5)
    const float* ln_w;
    const float* ln_b;
    // EPI_BIAS_POS: + pos[(r % W) % per]; EPI_BIAS_RES: + R[r][n] (ldr = N)
    const float* pos;
    int per;
    const float* R;
    // EPI_DOTS: f2 = z + slot_emb + acc + bias, dots with tw [T][N] and cw [T][N] into
    // part[r][block][2T]
    const float* z;
    const float* tw;
    const float* cw;
    float* part;
    int T;
    // split K (gridDim.z > 1): kc_per chunks of KC per split, raw sums into Cs [gridDim.z][M][N]
    int kc_per;
    float* Cs;
};

// split-K epilogue: C[r][n] = sum over splits of Cs[s][r][n] + bias[n] (+ pos[(r % W) % per][n]) (+ R[r][n]),
// the splits added in order
template <int EPI>
__global__ void __launch_bounds__(NT) k_head_splitk(GemmP p, int splits) {
    const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (i >= (int64_t)p.M * p.N) return;
    const int r = (int)(i / p.N), n = (int)(i % p.N);
    // eight splits' sums loaded before the first is added (indices past the last split read it
    // again, unused), added in split order
    const int64_t mn = (int64_t)p.M * p.N;
    float x = 0.0f;
    for (int s0 = 0; s0 < splits; s0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p.Cs[(int64_t)min(s0 + u, splits - 1) * mn + i];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float xs = x + v[u];
            x = s0 + u < splits ? xs : x;
        }
    }
    x += p.bias[n];
    if constexpr (EPI == EPI_BIAS_POS) x += p.pos[(int64_t)((r % p.W) % p.per) * p.N + n];
    if constexpr (EPI == EPI_BIAS_RES) x += p.R[(int64_t)r * p.N + n];
    if constexpr (EPI == EPI_BIAS_RELU) x = fmaxf(x, 0.0f);
    p.C[(int64_t)r * p.ldc + n] = x;
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// One workgroup = a TM x TN tile of C, the four waves its 32 x 32 quarters on v_mfma_f32_32x32x2_f32
// (float32 operands and sums).  Lane l of a wave supplies A[l % 32][k + l / 32] and B[k + l / 32][l % 32]
// and holds C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32] in accumulator v.  K runs in chunks of KC staged
// through LDS: A rows as they are (the prologue applied on the way: slot embedding or LayerNorm),
// the weights transposed to [k][n] with one column per lane.  VEC: K % 4 == 0 and the weights 16-byte
// aligned (each lane's four k of a column in one 16-byte load).
template <int PRO, int EPI, bool VEC>
__global__ void __launch_bounds__(NT) k_head_gemm(GemmP p) {
    __shared__ float sA[TM][KC + 1];
    __shared__ float sB[KC][TN + 32];          // rows 32 banks apart: the two half-waves' k rows
    __shared__ float sMean[TM], sRstd[TM];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;   // the wave's quarter of the tile
    const int l32 = lane & 31, h = lane >> 5;
    const int r0 = blockIdx.x * TM, n0 = blockIdx.y * TN;
    if constexpr (PRO == PRO_LN) {
        // mean and 1/std of the tile's rows (biased variance, as torch's layer_norm), in two passes
        // over the row: the mean, then the mean square deviation; 4 lanes per row
        // (lane l4 of a row takes its quads l4, l4 + 4, ..., LQ of them per round, all loaded before
        // the first is added; K % 4 == 0 for these products; rows past M read row M - 1, unused)
        const int rr = tid >> 2, l4 = tid & 3;
        const int r = r0 + rr;
        const float4* row4 = (const float4*)(p.A + (int64_t)min(r, p.M - 1) * p.K);
        const int nq = p.K >> 2;
        constexpr int LQ = 8;
        float s = 0.0f;
        for (int q0 = l4; q0 < nq; q0 += 4 * LQ) {
            float4 x[LQ];
#pragma unroll
            for (int i = 0; i < LQ; ++i) x[i] = row4[min(q0 + 4 * i, nq - 1)];
#pragma unroll
            for (int i = 0; i < LQ; ++i)
                if (q0 + 4 * i < nq) s += x[i].x + x[i].y + x[i].z + x[i].w;
        }
        s += __shfl_xor(s, 2, 4);
        s += __shfl_xor(s, 1, 4);
        const float mean = s / (float)p.K;
        float ss = 0.0f;
        for (int q0 = l4; q0 < nq; q0 += 4 * LQ) {
            float4 x[LQ];
#pragma unroll
            for (int i = 0; i < LQ; ++i) x[i] = row4[min(q0 + 4 * i, nq - 1)];
#pragma unroll
            for (int i = 0; i < LQ; ++i)
                if (q0 + 4 * i < nq) {
                    const float a = x[i].x - mean, b = x[i].y - mean, c = x[i].z - mean, d = x[i].w - mean;
                    ss = __builtin_fmaf(a, a, ss);
                    ss = __builtin_fmaf(b, b, ss);
                    ss = __builtin_fmaf(c, c, ss);
                    ss = __builtin_fmaf(d, d, ss);
                }
        }
        ss += __shfl_xor(ss, 2, 4);
        ss += __shfl_xor(ss, 1, 4);
        if (l4 == 0) {
            sMean[rr] = mean;
            sRstd[rr] = 1.0f / sqrtf(ss / (float)p.K + 1e-5f);
        }
        __syncthreads();
    }
    // this thread stages A rows tid / KC + (NT / KC) j at column tid % KC of each chunk: the rows'
    // addresses (and their slot embedding rows) are fixed for the whole K loop
    constexpr int AR = TM * KC / NT;
    static_assert(TM * KC % NT == 0 && NT % KC == 0 && TM == 64 && TN == 64, "staging");
    // Every load of the K loop is unconditional, from an address clamped into its table (rows past M
    // read row M - 1, columns past the split's end its last column, an absent slot row 0), and the
    // value is zeroed afterwards by an integer mask (a select of a loaded value is turned back into a
    // branch around the load, and a load under a branch waits for every load in flight before it).
    const int akk = tid % KC, ar0 = tid / KC;
    const float* arow[AR];
    const float* srow[AR];
    uint32_t rmask = 0u, smask = 0u;                 // bit j: row j is inside M / has a slot row
#pragma unroll
    for (int j = 0; j < AR; ++j) {
        const int r = r0 + ar0 + (NT / KC) * j;
        if (r < p.M) rmask |= 1u << j;
        arow[j] = p.A + (int64_t)min(r, p.M - 1) * p.K;
        srow[j] = nullptr;
        if constexpr (PRO == PRO_SLOT) {
            const int sl = r < p.M ? p.slot_of[r % p.W] : -1;
            const bool has = (unsigned)sl < (unsigned)p.S;
            if (has) smask |= 1u << j;
            srow[j] = p.slot_emb + (int64_t)(has ? sl : 0) * p.K;
        }
    }
    // split K: block z of gridDim.z takes chunks [z kc_per, (z + 1) kc_per)
    int kbeg = 0, kend = p.K;
    if (gridDim.z > 1) {
        kbeg = blockIdx.z * p.kc_per * KC;
        kend = min(p.K, kbeg + p.kc_per * KC);
    }
    const int bn = tid % TN, n = n0 + bn, bq = tid / TN;       // weights: column bn, k quads bq + 4 u
    constexpr int BQ = KC / 16;                                  // quads per thread and chunk
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    // chunk k0's values are fetched into registers (ra, rb) one chunk ahead: their loads are in flight
    // while the previous chunk's MFMAs run
    float ra[AR], rs[PRO == PRO_SLOT ? AR : 1];
    float4 rb[BQ];
    float rlw = 0.0f, rlb = 0.0f;                    // PRO_LN: the column's ln_w, ln_b
    const float* bcol = p.Bw + (int64_t)min(n, p.N - 1) * p.K;
    const bool nin = n < p.N;
    auto keep = [](float x, bool on) INLINE_H {
        uint32_t m = on ? ~0u : 0u;
        asm volatile("" : "+v"(m));                  // (opaque: the AND is not turned into a select)
        return __uint_as_float(__float_as_uint(x) & m);
    };
    // the raw values of chunk k0 (in flight during the previous chunk's MFMAs)
    auto fetch = [&](int k0) {
        const int kc = min(k0 + akk, kend - 1);
        if constexpr (PRO == PRO_LN) {
            rlw = p.ln_w[kc];
            rlb = p.ln_b[kc];
        }
#pragma unroll
        for (int j = 0; j < AR; ++j) {
            ra[j] = arow[j][kc];
            if constexpr (PRO == PRO_SLOT) rs[j] = srow[j][kc];
        }
#pragma unroll
        for (int u = 0; u < BQ; ++u) {
            const int kq = k0 + 4 * (bq + 4 * u);
            if constexpr (VEC) {
                // K % 4 == 0, so kend (a multiple of KC, or K) is too: kend - 4 starts a whole quad
                rb[u] = *(const float4*)(bcol + min(kq, kend - 4));
            } else {
                rb[u] = make_float4(bcol[min(kq + 0, kend - 1)], bcol[min(kq + 1, kend - 1)],
                                    bcol[min(kq + 2, kend - 1)], bcol[min(kq + 3, kend - 1)]);
            }
        }
    };
    fetch(kbeg);
    for (int k0 = kbeg; k0 < kend; k0 += KC) {
        // stage chunk k0: the values outside the matrix or the split zeroed, the prologue applied
        const int k = k0 + akk;
        const bool kin = k < kend;
#pragma unroll
        for (int j = 0; j < AR; ++j) {
            const int rr = ar0 + (NT / KC) * j;
            const bool on = kin && ((rmask >> j) & 1u);
            float v = ra[j];
            if constexpr (PRO == PRO_SLOT) {
                const float vs = v + rs[j];
                v = ((smask >> j) & 1u) ? vs : v;
            }
            v = keep(v, on);
            if constexpr (PRO == PRO_LN) {
                const float y = (v - sMean[rr]) * sRstd[rr] * rlw + rlb;
                v = on ? y : v;
            }
            sA[rr][akk] = v;
        }
#pragma unroll
        for (int u = 0; u < BQ; ++u) {
            const int q = bq + 4 * u;
            const int kq = k0 + 4 * q;
            float4 w = rb[u];
            if constexpr (VEC) {
                const bool on = nin && kq < kend;
                w = make_float4(keep(w.x, on), keep(w.y, on), keep(w.z, on), keep(w.w, on));
            } else {
                w = make_float4(keep(w.x, nin && kq + 0 < kend), keep(w.y, nin && kq + 1 < kend),
                                keep(w.z, nin && kq + 2 < kend), keep(w.w, nin && kq + 3 < kend));
            }
            sB[4 * q + 0][bn] = w.x;
            sB[4 * q + 1][bn] = w.y;
            sB[4 * q + 2][bn] = w.z;
            sB[4 * q + 3][bn] = w.w;
        }
        __syncthreads();
        if (k0 + KC < kend) fetch(k0 + KC);
#pragma unroll
        for (int kk = 0; kk < KC; kk += 2) {
            const float av = sA[32 * wr + l32][kk + h];
            const float bv = sB[kk + h][32 * wc + l32];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    const int n_out = n0 + 32 * wc + l32;
    if (gridDim.z > 1) {
        // split K: raw sums into the split's slice of Cs; k_head_splitk adds them and applies the epilogue
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = r0 + 32 * wr + 8 * (v >> 2) + 4 * h + (v & 3);
            if (r < p.M && n_out < p.N) p.Cs[((int64_t)blockIdx.z * p.M + r) * p.N + n_out] = acc[v];
        }
        return;
    }
    // the epilogues' loads, too, are issued together from clamped addresses before any is used
    const int nc = min(n_out, p.N - 1);
    const float bias_n = p.bias[nc];
    if constexpr (EPI != EPI_DOTS) {
        float ex[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int rc = min(r0 + 32 * wr + 8 * (v >> 2) + 4 * h + (v & 3), p.M - 1);
            ex[v] = 0.0f;
            if constexpr (EPI == EPI_BIAS_POS) ex[v] = p.pos[(int64_t)((rc % p.W) % p.per) * p.N + nc];
            if constexpr (EPI == EPI_BIAS_RES) ex[v] = p.R[(int64_t)rc * p.N + nc];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = r0 + 32 * wr + 8 * (v >> 2) + 4 * h + (v & 3);
            if (r >= p.M || n_out >= p.N) continue;
            float x = acc[v] + bias_n;
            if constexpr (EPI == EPI_BIAS_POS || EPI == EPI_BIAS_RES) x += ex[v];
            if constexpr (EPI == EPI_BIAS_RELU) x = fmaxf(x, 0.0f);
            p.C[(int64_t)r * p.ldc + n_out] = x;
        }
    } else {
        // f2 = z + slot_emb + acc + bias into LDS (the A tile's space), the attention and classifier
        // weights of these 64 columns beside it; then 4 lanes per row take 16 columns each and the
        // row's dots are summed over the 4 lanes
        __shared__ float sF[TM][TN + 1];
        __shared__ float sW[2 * TMAX][TN];
        // z and the slot indices of the lane's 16 rows, then their slot embedding rows (row 0 for
        // an absent slot, unused), then f2 = ((acc + b) + z) + (slot embedding or +0)
        int slv[16];
        float zv[16], sev[16];
        uint32_t hasm = 0u;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int rc = min(r0 + 32 * wr + 8 * (v >> 2) + 4 * h + (v & 3), p.M - 1);
            slv[v] = p.slot_of[rc % p.W];
            zv[v] = p.z[(int64_t)rc * p.N + nc];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const bool has = (unsigned)slv[v] < (unsigned)p.S;
            if (has) hasm |= 1u << v;
            sev[v] = p.slot_emb[(int64_t)(has ? slv[v] : 0) * p.N + nc];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int i = 32 * wr + 8 * (v >> 2) + 4 * h + (v & 3), r = r0 + i;
            const float x = acc[v] + bias_n + zv[v] + keep(sev[v], (hasm >> v) & 1u);
            sF[i][32 * wc + l32] = keep(x, r < p.M && n_out < p.N);
        }
        // the attention and classifier weights of these columns (rows T of tw, then T of cw)
        constexpr int WI = 2 * TMAX * TN / NT;
        float wv[WI];
#pragma unroll
        for (int u = 0; u < WI; ++u) {
            const int i = tid + u * NT, q = min(i / TN, 2 * p.T - 1), c = i % TN;
            const float* src = q < p.T ? p.tw + (int64_t)q * p.N : p.cw + (int64_t)(q - p.T) * p.N;
            wv[u] = src[min(n0 + c, p.N - 1)];
        }
#pragma unroll
        for (int u = 0; u < WI; ++u) {
            const int i = tid + u * NT, q = i / TN, c = i % TN;
            if (i < 2 * p.T * TN) sW[q][c] = keep(wv[u], n0 + c < p.N);
        }
        __syncthreads();
        const int rr = tid >> 2, c0 = 16 * (tid & 3), r = r0 + rr;
        for (int t = 0; t < p.T; ++t) {
            float da = 0.0f, dc = 0.0f;
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const float x = sF[rr][c0 + c];
                da = __builtin_fmaf(x, sW[t][c0 + c], da);
                dc = __builtin_fmaf(x, sW[p.T + t][c0 + c], dc);
            }
            da += __shfl_xor(da, 2, 4);
            da += __shfl_xor(da, 1, 4);
            dc += __shfl_xor(dc, 2, 4);
            dc += __shfl_xor(dc, 1, 4);
            if ((tid & 3) == 0 && r < p.M) {
                float* dst = p.part + ((int64_t)r * gridDim.y + blockIdx.y) * 2 * p.T;
                dst[t] = da;
                dst[p.T + t] = dc;
            }
        }
    }
}

struct AttnP {
    const float* qkv;      // [B*W][3 CD]
    const uint8_t* valid;  // [B][W] 1 = key of a present slot (absent slots are not keys)
    float* out;            // [B*W][CD]
    int W, CD, heads;
};

// One workgroup per (study, head, 16 queries), 16 lanes per query: softmax(q k^T / sqrt(dh)) v over
// the keys of present slots (all keys when no slot of the study is present).  Lane l of a query scores
// keys l, l + 16, ... with full 64-dim dots (q in registers), the maximum and the sum are reduced over
// the 16 lanes, the unnormalised weights go to LDS, and lane l then accumulates output dims 4l .. 4l + 3
// over all keys.
constexpr int AQ = 16;   // queries per workgroup
__global__ void __launch_bounds__(NT) k_head_attn(AttnP p) {
    constexpr int DH = 64, LQ = NT / AQ, KPL = WMAX / LQ;
    static_assert(LQ == 16 && DH == 4 * LQ, "attention lanes");
    __shared__ float4 sK[WMAX][DH / 4 + 1];
    __shared__ float4 sV[WMAX][DH / 4];
    __shared__ float sP[AQ][WMAX];
    __shared__ uint8_t sKey[WMAX];
    __shared__ int sAny;
    const int b = blockIdx.x, h = blockIdx.y, q0 = blockIdx.z * AQ;
    const int ld = 3 * p.CD;
    const float* base = p.qkv + (int64_t)b * p.W * ld;
    {
        // the keys and values of the study, all loads issued before the first LDS store (items past
        // W * 16 read the last one again and fill rows W .. WMAX - 1, which no score or output reads)
        constexpr int KV = WMAX * (DH / 4) / NT;
        float4 kv[2 * KV];
        const int n = p.W * (DH / 4);
#pragma unroll
        for (int u = 0; u < KV; ++u) {
            const int i = min((int)threadIdx.x + u * NT, n - 1), w = i / (DH / 4), d4 = i % (DH / 4);
            kv[2 * u] = *(const float4*)(base + (int64_t)w * ld + p.CD + h * DH + 4 * d4);
            kv[2 * u + 1] = *(const float4*)(base + (int64_t)w * ld + 2 * p.CD + h * DH + 4 * d4);
        }
        static_assert(KV * NT == WMAX * (DH / 4), "one item per row and quad of sK / sV");
#pragma unroll
        for (int u = 0; u < KV; ++u) {
            const int i = (int)threadIdx.x + u * NT, w = i / (DH / 4), d4 = i % (DH / 4);
            sK[w][d4] = kv[2 * u];
            sV[w][d4] = kv[2 * u + 1];
        }
    }
    if (threadIdx.x == 0) sAny = 0;
    __syncthreads();
    for (int w = threadIdx.x; w < p.W; w += NT)
        if (p.valid[(int64_t)b * p.W + w]) atomicOr(&sAny, 1);
    __syncthreads();
    for (int w = threadIdx.x; w < p.W; w += NT) sKey[w] = sAny ? p.valid[(int64_t)b * p.W + w] : 1;
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)DH);
    const int ql = threadIdx.x / LQ, l = threadIdx.x % LQ, qi = q0 + ql;
    const bool act = qi < p.W;
    // (a query past W reads the last one: its scores and output are computed and not stored)
    const int qc = min(qi, p.W - 1);
    float4 q[DH / 4];
#pragma unroll
    for (int d4 = 0; d4 < DH / 4; ++d4) {
        const float4 v = *(const float4*)(base + (int64_t)qc * ld + h * DH + 4 * d4);
        q[d4] = make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
    }
    float sc[KPL];
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        const int j = l + LQ * m;
        sc[m] = -INFINITY;
        if (j < p.W && sKey[j]) {
            float s = 0.0f;
#pragma unroll
            for (int d4 = 0; d4 < DH / 4; ++d4) {
                const float4 k = sK[j][d4];
                s = __builtin_fmaf(q[d4].x, k.x, s);
                s = __builtin_fmaf(q[d4].y, k.y, s);
                s = __builtin_fmaf(q[d4].z, k.z, s);
                s = __builtin_fmaf(q[d4].w, k.w, s);
            }
            sc[m] = s;
            mx = fmaxf(mx, s);
        }
    }
#pragma unroll
    for (int d = LQ / 2; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d, LQ));
    float sum = 0.0f;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        const int j = l + LQ * m;
        if (j < p.W) {
            const float e = sc[m] == -INFINITY ? 0.0f : expf(sc[m] - mx);
            sum += e;
            sP[ql][j] = e;
        }
    }
#pragma unroll
    for (int d = LQ / 2; d >= 1; d >>= 1) sum += __shfl_xor(sum, d, LQ);
    __syncthreads();
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j = 0; j < p.W; ++j) {
        const float e = sP[ql][j];
        const float4 v = sV[j][l];
        o.x = __builtin_fmaf(e, v.x, o.x);
        o.y = __builtin_fmaf(e, v.y, o.y);
        o.z = __builtin_fmaf(e, v.z, o.z);
        o.w = __builtin_fmaf(e, v.w, o.w);
    }
    if (act) {
        const float inv = 1.0f / sum;
        *(float4*)(p.out + ((int64_t)b * p.W + qi) * p.CD + h * DH + 4 * l) =
            make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    }
}

// The partial dots of every (window row, value) summed over the column blocks of the dots product,
// 8 loads in flight: sums[r][q] (q < T: attention logit, + attn_b; else the classifier dot)
__global__ void __launch_bounds__(NT) k_head_dotsum(const float* part, const float* attn_b, float* sums,
                                                    int M, int T, int nblk) {
    const int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (i >= (int64_t)M * 2 * T) return;
    const int64_t r = i / (2 * T);
    const int q = (int)(i % (2 * T));
    const float* pr = part + r * nblk * 2 * T + q;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    int k = 0;
    for (; k + 8 <= nblk; k += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u] += pr[(k + u) * 2 * T];
    }
    for (; k < nblk; ++k) acc[0] += pr[k * 2 * T];
    const float sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    sums[i] = q < T ? sum + attn_b[q] : sum;
}

struct PoolP {
    const float* sums;     // [B*W][2T]
    const uint8_t* valid;  // [B][W]
    const float* cls_b;    // [T]
    float* logits;         // [B][T]
    int W, T;
};

// One workgroup per study: a[w][t] = attn(f2[w]) + b (masked to -inf for absent slots; all zeros
// when no slot is present), softmax over the windows, logits[t] = sum_w a[w][t] s[w][t] + cls_b[t].
__global__ void __launch_bounds__(NT) k_head_pool(PoolP p) {
    __shared__ float sA[WMAX][TMAX], sS[WMAX][TMAX];
    const int b = blockIdx.x;
    {
        // all of the study's sums loaded before the first LDS store (past W * 2T: the last, unused)
        constexpr int PN = WMAX * 2 * TMAX / NT;
        const int n = p.W * 2 * p.T;
        float v[PN];
#pragma unroll
        for (int u = 0; u < PN; ++u) v[u] = p.sums[(int64_t)b * n + min((int)threadIdx.x + u * NT, n - 1)];
#pragma unroll
        for (int u = 0; u < PN; ++u) {
            const int i = (int)threadIdx.x + u * NT, w = i / (2 * p.T), q = i % (2 * p.T);
            if (i < n) {
                if (q < p.T)
                    sA[w][q] = v[u];
                else
                    sS[w][q - p.T] = v[u];
            }
        }
    }
    __shared__ uint8_t sV[WMAX];
    __shared__ int sAny;
    if (threadIdx.x == 0) sAny = 0;
    __syncthreads();
    for (int w = threadIdx.x; w < p.W; w += NT) {
        sV[w] = p.valid[(int64_t)b * p.W + w];
        if (sV[w]) atomicOr(&sAny, 1);
    }
    __syncthreads();
    // 16 lanes per finding t, lane l taking windows l, l + 16, ...: maximum, then the sums, reduced
    // over the 16 lanes
    const int t = threadIdx.x / 16, l = threadIdx.x % 16;
    const bool any = sAny != 0;
    float mx = -INFINITY;
    if (t < p.T)
        for (int w = l; w < p.W; w += 16) mx = fmaxf(mx, any ? (sV[w] ? sA[w][t] : -INFINITY) : 0.0f);
#pragma unroll
    for (int d = 8; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d, 16));
    float sum = 0.0f, acc = 0.0f;
    if (t < p.T)
        for (int w = l; w < p.W; w += 16) {
            const float a = any ? (sV[w] ? sA[w][t] : -INFINITY) : 0.0f;
            const float e = expf(a - mx);
            sum += e;
            acc = __builtin_fmaf(e, sS[w][t], acc);
        }
#pragma unroll
    for (int d = 8; d >= 1; d >>= 1) {
        sum += __shfl_xor(sum, d, 16);
        acc += __shfl_xor(acc, d, 16);
    }
    if (t < p.T && l == 0) p.logits[(int64_t)b * p.T + t] = acc / sum + p.cls_b[t];
}

// valid[b][w] = slot_mask[b][slot_of[w]] (0 for a slot outside 0 .. S-1)
__global__ void __launch_bounds__(NT) k_head_valid(const uint8_t* slot_mask, const int32_t* slot_of,
                                                   uint8_t* valid, int B, int W, int S) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i >= B * W) return;
    const int sl = slot_of[i % W];
    valid[i] = (unsigned)sl < (unsigned)S && slot_mask[(int64_t)(i / W) * S + sl] ? 1 : 0;
}

#define HREQ(cond, msg) \
    do { if (!(cond)) return d8s_host_fail((int)hipErrorInvalidValue, std::string(what) + ": " + (msg)); } while (0)

// K split of a product of M rows, N columns and depth K: enough workgroups for the chip (about 512)
// when the M x N tiles alone are few
struct Split {
    int splits, kc_per;
};

Split split_plan(int64_t M, int N, int K) {
    const int chunks = (K + KC - 1) / KC;
    const int64_t base = (M + TM - 1) / TM * ((N + TN - 1) / TN);
    if (base >= 256 || chunks < 2) return {1, chunks};
    const int want = (int)std::min<int64_t>(chunks, (512 + base - 1) / base);
    const int kc = (chunks + want - 1) / want;
    return {(chunks + kc - 1) / kc, kc};
}

struct Ws {
    float *h, *qkv, *att, *h1, *u, *h2, *part, *sums, *cs;
    uint8_t* valid;
    uint64_t bytes;
};

Ws carve(const D8sHeadArgs* a, char* base) {
    Ws w{};
    const int64_t M = (int64_t)a->B * a->W;
    const int nblk = (a->D + TN - 1) / TN;
    uint64_t off = 0;
    auto take = [&](uint64_t n) {
        char* p = base ? base + off : nullptr;
        off += (n + 255) / 256 * 256;
        return p;
    };
    const bool ctx = true;
    w.h = (float*)take(ctx ? 4ull * M * a->CD : 0);
    w.qkv = (float*)take(ctx ? 12ull * M * a->CD : 0);
    w.att = (float*)take(ctx ? 4ull * M * a->CD : 0);
    w.h1 = (float*)take(ctx ? 4ull * M * a->CD : 0);
    w.u = (float*)take(ctx ? 4ull * M * a->FF : 0);
    w.h2 = (float*)take(ctx ? 4ull * M * a->CD : 0);
    w.part = (float*)take(4ull * M * nblk * 2 * a->T);
    w.sums = (float*)take(4ull * M * 2 * a->T);
    uint64_t cs = 0;
    const int dims[5][2] = {{a->CD, a->D}, {3 * a->CD, a->CD}, {a->CD, a->CD}, {a->FF, a->CD}, {a->CD, a->FF}};
    for (const auto& d : dims) {
        const Split sp = split_plan(M, d[0], d[1]);
        if (sp.splits > 1) cs = std::max<uint64_t>(cs, 4ull * sp.splits * M * d[0]);
    }
    w.cs = (float*)take(cs);
    w.valid = (uint8_t*)take((uint64_t)M);
    w.bytes = off;
    return w;
}

// whether a product's weights can be read as 16-byte quads along K
bool gemm_vec(const GemmP& g) { return (g.K & 3) == 0 && ((uintptr_t)g.Bw & 15) == 0; }

// one context-layer product, split over K when its tiles alone are too few for the chip
template <int PRO, int EPI>
void launch_gemm(GemmP g, float* cs, hipStream_t st) {
    static_assert(EPI != EPI_DOTS, "the dots epilogue is not split");
    const Split sp = split_plan(g.M, g.N, g.K);
    const dim3 grid((g.M + TM - 1) / TM, (g.N + TN - 1) / TN, sp.splits);
    g.kc_per = sp.kc_per;
    g.Cs = cs;
    if (gemm_vec(g))
        k_head_gemm<PRO, EPI, true><<<grid, NT, 0, st>>>(g);
    else
        k_head_gemm<PRO, EPI, false><<<grid, NT, 0, st>>>(g);
    if (sp.splits > 1) {
        const int64_t n = (int64_t)g.M * g.N;
        k_head_splitk<EPI><<<(unsigned)((n + NT - 1) / NT), NT, 0, st>>>(g, sp.splits);
    }
}

}  // namespace

extern "C" int d8s_head_workspace(const D8sHeadArgs* a, uint64_t* bytes) {
    const char* what = "d8s_head_workspace";
    HREQ(a != nullptr && bytes != nullptr, "null arguments");
    HREQ(a->B >= 1 && a->W >= 1 && a->D >= 1 && a->T >= 1, "bad sizes");
    *bytes = carve(a, nullptr).bytes;
    return 0;
}

namespace {

// Checks the arguments (everything but the workspace) and returns the workspace layout's size.
int head_check(const D8sHeadArgs* a, const char* what) {
    HREQ(a != nullptr, "null arguments");
    HREQ(a->z && a->slot_of && a->slot_mask && a->slot_emb && a->attn_w && a->attn_b && a->cls_w &&
         a->cls_b && a->logits, "null pointer");
    HREQ(a->B >= 1 && a->B < 65536, "B must be 1 .. 65535");
    HREQ(a->W >= 1 && a->W <= WMAX, "W must be 1 .. 128 windows per study");
    HREQ(a->D >= 1 && a->S >= 1 && a->T >= 1 && a->T <= TMAX, "bad D, S or T (T <= 16)");
    HREQ(a->ctx_layers == 1, "ctx_layers must be 1 (one context layer)");
    {
        HREQ(a->ctx_in_w && a->ctx_in_b && a->ctx_pos && a->in_proj_w && a->in_proj_b && a->out_proj_w &&
             a->out_proj_b && a->ln1_w && a->ln1_b && a->ln2_w && a->ln2_b && a->ff1_w && a->ff1_b &&
             a->ff2_w && a->ff2_b && a->ctx_out_w && a->ctx_out_b, "null context weight");
        HREQ(a->heads >= 1 && a->CD == 64 * a->heads, "context width must be 64 x heads");
        HREQ(a->FF >= 1 && a->PER >= 1, "bad FF or PER");
    }
    HREQ((int64_t)a->B * a->W * a->D < (1ll << 31), "too many values");
    return 0;
}

// The launch sequence of the head over the workspace `ws` (laid out by carve).
void head_run(const D8sHeadArgs* a, char* ws, hipStream_t st) {
    const Ws w = carve(a, ws);
    const int M = a->B * a->W;
    const int nblk = (a->D + TN - 1) / TN;
    k_head_valid<<<(M + NT - 1) / NT, NT, 0, st>>>(a->slot_mask, a->slot_of, w.valid, a->B, a->W, a->S);
    {
        GemmP g{};
        g.M = M;
        g.W = a->W;
        g.S = a->S;
        g.slot_of = a->slot_of;
        g.slot_emb = a->slot_emb;
        // 1. h = (z + slot_emb) ctx_in^T + b + ctx_pos[w % per]
        g.A = a->z; g.Bw = a->ctx_in_w; g.bias = a->ctx_in_b; g.C = w.h;
        g.N = a->CD; g.K = a->D; g.ldc = a->CD; g.pos = a->ctx_pos; g.per = a->PER;
        launch_gemm<PRO_SLOT, EPI_BIAS_POS>(g, w.cs, st);
        // 2. qkv = LN1(h) in_proj^T + b
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.h; g.Bw = a->in_proj_w; g.bias = a->in_proj_b; g.C = w.qkv;
        g.N = 3 * a->CD; g.K = a->CD; g.ldc = 3 * a->CD; g.ln_w = a->ln1_w; g.ln_b = a->ln1_b;
        launch_gemm<PRO_LN, EPI_BIAS>(g, w.cs, st);
        // 3. attention per (study, head)
        AttnP at{w.qkv, w.valid, w.att, a->W, a->CD, a->heads};
        k_head_attn<<<dim3(a->B, a->heads, (a->W + AQ - 1) / AQ), NT, 0, st>>>(at);
        // 4. h1 = h + att out_proj^T + b
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.att; g.Bw = a->out_proj_w; g.bias = a->out_proj_b; g.C = w.h1;
        g.N = a->CD; g.K = a->CD; g.ldc = a->CD; g.R = w.h;
        launch_gemm<PRO_NONE, EPI_BIAS_RES>(g, w.cs, st);
        // 5. u = relu(LN2(h1) ff1^T + b)
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.h1; g.Bw = a->ff1_w; g.bias = a->ff1_b; g.C = w.u;
        g.N = a->FF; g.K = a->CD; g.ldc = a->FF; g.ln_w = a->ln2_w; g.ln_b = a->ln2_b;
        launch_gemm<PRO_LN, EPI_BIAS_RELU>(g, w.cs, st);
        // 6. h2 = h1 + u ff2^T + b
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.u; g.Bw = a->ff2_w; g.bias = a->ff2_b; g.C = w.h2;
        g.N = a->CD; g.K = a->FF; g.ldc = a->CD; g.R = w.h1;
        launch_gemm<PRO_NONE, EPI_BIAS_RES>(g, w.cs, st);
    }
    // 7. f2 = z + slot_emb + h2 ctx_out^T + b, partial dots with attn.weight and cls_w
    GemmP g{};
    g.M = M; g.W = a->W; g.S = a->S; g.slot_of = a->slot_of; g.slot_emb = a->slot_emb;
    g.N = a->D; g.z = a->z; g.tw = a->attn_w; g.cw = a->cls_w; g.part = w.part; g.T = a->T;
    g.A = w.h2; g.Bw = a->ctx_out_w; g.bias = a->ctx_out_b; g.K = a->CD;
    if (gemm_vec(g))
        k_head_gemm<PRO_NONE, EPI_DOTS, true><<<dim3((M + TM - 1) / TM, nblk), NT, 0, st>>>(g);
    else
        k_head_gemm<PRO_NONE, EPI_DOTS, false><<<dim3((M + TM - 1) / TM, nblk), NT, 0, st>>>(g);
    // 8. pooling
    const int64_t nsum = (int64_t)M * 2 * a->T;
    k_head_dotsum<<<(unsigned)((nsum + NT - 1) / NT), NT, 0, st>>>(w.part, a->attn_b, w.sums, M, a->T, nblk);
    PoolP pp{w.sums, w.valid, a->cls_b, a->logits, a->W, a->T};
    k_head_pool<<<a->B, NT, 0, st>>>(pp);
}

}  // namespace

extern "C" int d8s_head(const D8sHeadArgs* a, void* stream) {
    const char* what = "d8s_head";
    if (int rc = head_check(a, what)) return rc;
    HREQ(a->workspace, "null workspace");
    HREQ(a->ws_bytes >= carve(a, nullptr).bytes, "workspace smaller than d8s_head_workspace()");
    head_run(a, (char*)a->workspace, (hipStream_t)stream);
    return d8s_host_launched(what);
}

// ---- the entry point that allocates nothing -------------------------------------------------------
// Its workspace is this array, one copy per GPU, held until the process ends.  Host code never uses
// the array's name as an address (on the host it is a stand-in, not device memory): the device
// address of each GPU's copy comes from hipGetSymbolAddress, looked up once per device with that
// device current, and is what the kernels receive.  Every call on a GPU shares that GPU's copy, so
// calls that overlap on one GPU (different streams, no ordering between them) race.
static __device__ __align__(256) unsigned char scratch[D8S_HEAD_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[MAX_DEVICES] = {};

// The device address of the current device's scratch; `stream` must belong to that device.
int scratch_ptr(hipStream_t stream, void** out, const char* what) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    HREQ(e == hipSuccess, std::string("hipGetDevice: ") + hipGetErrorString(e));
    HREQ(dev >= 0 && dev < MAX_DEVICES, "device ordinal out of range");
    if (stream != nullptr) {
        hipDevice_t sdev = -1;
        e = hipStreamGetDevice(stream, &sdev);
        HREQ(e == hipSuccess, std::string("hipStreamGetDevice: ") + hipGetErrorString(e));
        HREQ(sdev == dev, "the stream belongs to another device than the current one");
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        HREQ(e == hipSuccess && p != nullptr,
             std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace

extern "C" int d8s_head_noalloc(const D8sHeadArgs* a, void* stream) {
    const char* what = "d8s_head_noalloc";
    if (int rc = head_check(a, what)) return rc;
    const uint64_t need = carve(a, nullptr).bytes;
    HREQ(need <= D8S_HEAD_SCRATCH_BYTES,
         "workspace of " + std::to_string(need) + " bytes exceeds the static scratch of " +
             std::to_string((unsigned long long)D8S_HEAD_SCRATCH_BYTES) + " bytes (fewer studies per call)");
    void* ws = nullptr;
    if (int rc = scratch_ptr((hipStream_t)stream, &ws, what)) return rc;
    head_run(a, (char*)ws, (hipStream_t)stream);
    return d8s_host_launched(what);
}
