// gfx950 kernels of the head that follows the encoder (the reference's `KneeBaseline` context and
// per-finding attention pooling, src/knee/models/baseline.py:870-932,954-977,1083-1170) and their C
// ABI, d8s_head (include/d8s_hip.h).
//
// Per study (W windows of D-dim encoder features, a few hundred KB) the head is a few small matrix
// products with row-wise normalisations around them; the PyTorch head is ~30 launches of tiny
// kernels.  Here it is 8 launches for all studies of a call, float32 throughout:
//   1. k_head_gemm<PRO_SLOT, EPI_BIAS_POS>: h = (z + slot_emb[slot]) ctx_in^T + b + ctx_pos[w % per]
//   2. k_head_gemm<PRO_LN, EPI_BIAS>:       qkv = LN1(h) in_proj^T + b
//   3. k_head_attn:                          per (study, head) softmax(q k^T / sqrt(dh), keys of
//                                            absent slots masked) v
//   4. k_head_gemm<PRO_NONE, EPI_BIAS_RES>:  h1 = h + att out_proj^T + b
//   5. k_head_gemm<PRO_LN, EPI_BIAS_RELU>:   u = relu(LN2(h1) ff1^T + b)
//   6. k_head_gemm<PRO_NONE, EPI_BIAS_RES>:  h2 = h1 + u ff2^T + b
//   7. k_head_gemm<PRO_NONE, EPI_DOTS>:      f2 = z + slot_emb + h2 ctx_out^T + b, and per 64-column
//                                            block the partial dots of f2 with attn.weight and cls_w
//   8. k_head_pool:                          per study: a = attn(f2) masked, softmax over windows,
//                                            logits = sum_w a (f2 . cls_w) + cls_b
// (one context layer: the final model's configuration.)  The pooled vector of the reference,
// sum_w a f2, is never formed: its dot with cls_w is sum_w a (f2 . cls_w), the same value up to the
// order of the float32 sums.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <string>

#include "d8s_hip.h"
#include "d8s_host.h"

#define DEV __device__ __forceinline__

namespace {

constexpr int NT = 256;
constexpr int TM = 16, TN = 64, KC = 64;     // GEMM tile: 16 rows x 64 columns, K in chunks of 64
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
    // PRO_SLOT: A row r gets + slot_emb[slot_of[r % W]]
    const float* slot_emb;
    const int32_t* slot_of;
    int W;
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
};

template <int PRO, int EPI>
__global__ void __launch_bounds__(NT) k_head_gemm(GemmP p) {
    __shared__ float sA[TM][KC + 1];
    __shared__ float sB[KC][TN + 4];
    __shared__ float sMean[TM], sRstd[TM];
    const int tid = threadIdx.x;
    const int ty = tid >> 4, tx = tid & 15;           // row ty, columns 4 tx .. 4 tx + 3
    const int r0 = blockIdx.x * TM, n0 = blockIdx.y * TN;
    if constexpr (PRO == PRO_LN) {
        // mean and 1/std of the tile's rows (biased variance, as torch's layer_norm), in two passes
        // over the row: the mean, then the mean square deviation
        const int r = r0 + ty;
        float s = 0.0f;
        if (r < p.M)
            for (int k = tx; k < p.K; k += 16) s += p.A[(int64_t)r * p.K + k];
#pragma unroll
        for (int d = 8; d >= 1; d >>= 1) s += __shfl_xor(s, d, 16);
        const float mean = s / (float)p.K;
        float ss = 0.0f;
        if (r < p.M)
            for (int k = tx; k < p.K; k += 16) {
                const float x = p.A[(int64_t)r * p.K + k] - mean;
                ss = __builtin_fmaf(x, x, ss);
            }
#pragma unroll
        for (int d = 8; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 16);
        if (tx == 0) {
            sMean[ty] = mean;
            sRstd[ty] = 1.0f / sqrtf(ss / (float)p.K + 1e-5f);
        }
        __syncthreads();
    }
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < p.K; k0 += KC) {
        // A tile [TM][KC]: 4 values per thread
        for (int i = tid; i < TM * KC; i += NT) {
            const int rr = i / KC, kk = i % KC;
            const int r = r0 + rr, k = k0 + kk;
            float v = 0.0f;
            if (r < p.M && k < p.K) {
                v = p.A[(int64_t)r * p.K + k];
                if constexpr (PRO == PRO_SLOT) v += p.slot_emb[(int64_t)p.slot_of[r % p.W] * p.K + k];
                if constexpr (PRO == PRO_LN) v = (v - sMean[rr]) * sRstd[rr] * p.ln_w[k] + p.ln_b[k];
            }
            sA[rr][kk] = v;
        }
        // B tile: weights [n0 .. n0 + TN)[k0 .. k0 + KC) transposed into sB[k][n]
        for (int i = tid; i < TN * KC; i += NT) {
            const int nn = i / KC, kk = i % KC;
            const int n = n0 + nn, k = k0 + kk;
            sB[kk][nn] = (n < p.N && k < p.K) ? p.Bw[(int64_t)n * p.K + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < KC; ++kk) {
            const float a = sA[ty][kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __builtin_fmaf(a, sB[kk][4 * tx + j], acc[j]);
        }
        __syncthreads();
    }
    const int r = r0 + ty;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + 4 * tx + j;
        v[j] = 0.0f;
        if (r >= p.M || n >= p.N) continue;
        float x = acc[j] + p.bias[n];
        if constexpr (EPI == EPI_BIAS_POS) x += p.pos[(int64_t)((r % p.W) % p.per) * p.N + n];
        if constexpr (EPI == EPI_BIAS_RES) x += p.R[(int64_t)r * p.N + n];
        if constexpr (EPI == EPI_BIAS_RELU) x = fmaxf(x, 0.0f);
        if constexpr (EPI == EPI_DOTS)
            x += p.z[(int64_t)r * p.N + n] + p.slot_emb[(int64_t)p.slot_of[r % p.W] * p.N + n];
        v[j] = x;
        if constexpr (EPI != EPI_DOTS) p.C[(int64_t)r * p.ldc + n] = x;
    }
    if constexpr (EPI == EPI_DOTS) {
        // partial dots of the row's 64 columns with the attention and classifier weights
        __shared__ float sDot[TM][16][2 * TMAX];
        for (int t = 0; t < p.T; ++t) {
            float da = 0.0f, dc = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = n0 + 4 * tx + j;
                if (n < p.N) {
                    da = __builtin_fmaf(v[j], p.tw[(int64_t)t * p.N + n], da);
                    dc = __builtin_fmaf(v[j], p.cw[(int64_t)t * p.N + n], dc);
                }
            }
            sDot[ty][tx][t] = da;
            sDot[ty][tx][TMAX + t] = dc;
        }
        __syncthreads();
        if (r < p.M)
            for (int q = tx; q < 2 * p.T; q += 16) {
                const int t = q < p.T ? q : TMAX + q - p.T;
                float s = 0.0f;
                for (int i = 0; i < 16; ++i) s += sDot[ty][i][t];
                p.part[((int64_t)r * gridDim.y + blockIdx.y) * 2 * p.T + q] = s;
            }
    }
}

struct AttnP {
    const float* qkv;      // [B*W][3 CD]
    const uint8_t* valid;  // [B][W] 1 = key of a present slot (absent slots are not keys)
    float* out;            // [B*W][CD]
    int W, CD, heads;
};

// One workgroup per (study, head): every thread owns query rows; softmax(q k^T / sqrt(dh)) v over the
// keys of present slots (all keys when no slot of the study is present).
__global__ void __launch_bounds__(NT) k_head_attn(AttnP p) {
    constexpr int DH = 64;
    __shared__ float sK[WMAX][DH + 1];
    __shared__ float sV[WMAX][DH + 1];
    __shared__ uint8_t sKey[WMAX];
    const int b = blockIdx.x, h = blockIdx.y;
    const int ld = 3 * p.CD;
    const float* base = p.qkv + (int64_t)b * p.W * ld;
    for (int i = threadIdx.x; i < p.W * DH; i += NT) {
        const int w = i / DH, d = i % DH;
        sK[w][d] = base[(int64_t)w * ld + p.CD + h * DH + d];
        sV[w][d] = base[(int64_t)w * ld + 2 * p.CD + h * DH + d];
    }
    int any = 0;
    for (int w = 0; w < p.W; ++w) any |= p.valid[(int64_t)b * p.W + w];
    for (int w = threadIdx.x; w < p.W; w += NT) sKey[w] = any ? p.valid[(int64_t)b * p.W + w] : 1;
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)DH);
    for (int qi = threadIdx.x; qi < p.W; qi += NT) {
        float q[DH];
#pragma unroll
        for (int d = 0; d < DH; ++d) q[d] = base[(int64_t)qi * ld + h * DH + d] * scale;
        float mx = -INFINITY;
        for (int j = 0; j < p.W; ++j) {
            if (!sKey[j]) continue;
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < DH; ++d) s = __builtin_fmaf(q[d], sK[j][d], s);
            mx = fmaxf(mx, s);
        }
        float sum = 0.0f, o[DH];
#pragma unroll
        for (int d = 0; d < DH; ++d) o[d] = 0.0f;
        for (int j = 0; j < p.W; ++j) {
            if (!sKey[j]) continue;
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < DH; ++d) s = __builtin_fmaf(q[d], sK[j][d], s);
            const float e = expf(s - mx);
            sum += e;
#pragma unroll
            for (int d = 0; d < DH; ++d) o[d] = __builtin_fmaf(e, sV[j][d], o[d]);
        }
        const float inv = 1.0f / sum;
        float* dst = p.out + ((int64_t)b * p.W + qi) * p.CD + h * DH;
#pragma unroll
        for (int d = 0; d < DH; ++d) dst[d] = o[d] * inv;
    }
}

struct PoolP {
    const float* part;     // [B*W][nblk][2T]
    const uint8_t* valid;  // [B][W]
    const float* attn_b;   // [T]
    const float* cls_b;    // [T]
    float* logits;         // [B][T]
    int W, T, nblk;
};

// One workgroup per study: a[w][t] = attn(f2[w]) + b (masked to -inf for absent slots; all zeros
// when no slot is present), softmax over the windows, logits[t] = sum_w a[w][t] s[w][t] + cls_b[t].
__global__ void __launch_bounds__(NT) k_head_pool(PoolP p) {
    __shared__ float sA[WMAX][TMAX], sS[WMAX][TMAX];
    const int b = blockIdx.x;
    for (int i = threadIdx.x; i < p.W * p.T; i += NT) {
        const int w = i / p.T, t = i % p.T;
        const float* pr = p.part + (int64_t)(b * p.W + w) * p.nblk * 2 * p.T;
        float sa = 0.0f, sc = 0.0f;
        for (int k = 0; k < p.nblk; ++k) {
            sa += pr[k * 2 * p.T + t];
            sc += pr[k * 2 * p.T + p.T + t];
        }
        sA[w][t] = sa + p.attn_b[t];
        sS[w][t] = sc;
    }
    __syncthreads();
    if (threadIdx.x < p.T) {
        const int t = threadIdx.x;
        int any = 0;
        for (int w = 0; w < p.W; ++w) any |= p.valid[(int64_t)b * p.W + w];
        float mx = -INFINITY;
        for (int w = 0; w < p.W; ++w) {
            const float a = any ? (p.valid[(int64_t)b * p.W + w] ? sA[w][t] : -INFINITY) : 0.0f;
            mx = fmaxf(mx, a);
        }
        float sum = 0.0f, acc = 0.0f;
        for (int w = 0; w < p.W; ++w) {
            const float a = any ? (p.valid[(int64_t)b * p.W + w] ? sA[w][t] : -INFINITY) : 0.0f;
            const float e = expf(a - mx);
            sum += e;
            acc = __builtin_fmaf(e, sS[w][t], acc);
        }
        p.logits[(int64_t)b * p.T + t] = acc / sum + p.cls_b[t];
    }
}

// valid[b][w] = slot_mask[b][slot_of[w]]
__global__ void __launch_bounds__(NT) k_head_valid(const uint8_t* slot_mask, const int32_t* slot_of,
                                                   uint8_t* valid, int B, int W, int S) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < B * W) valid[i] = slot_mask[(int64_t)(i / W) * S + slot_of[i % W]] ? 1 : 0;
}

#define HREQ(cond, msg) \
    do { if (!(cond)) return d8s_host_fail((int)hipErrorInvalidValue, std::string(what) + ": " + (msg)); } while (0)

struct Ws {
    float *h, *qkv, *att, *h1, *u, *h2, *part;
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
    w.valid = (uint8_t*)take((uint64_t)M);
    w.bytes = off;
    return w;
}

}  // namespace

extern "C" int d8s_head_workspace(const D8sHeadArgs* a, uint64_t* bytes) {
    const char* what = "d8s_head_workspace";
    HREQ(a != nullptr && bytes != nullptr, "null arguments");
    HREQ(a->B >= 1 && a->W >= 1 && a->D >= 1 && a->T >= 1, "bad sizes");
    *bytes = carve(a, nullptr).bytes;
    return 0;
}

extern "C" int d8s_head(const D8sHeadArgs* a, void* stream) {
    const char* what = "d8s_head";
    HREQ(a != nullptr, "null arguments");
    HREQ(a->z && a->slot_of && a->slot_mask && a->slot_emb && a->attn_w && a->attn_b && a->cls_w &&
         a->cls_b && a->logits && a->workspace, "null pointer");
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
    const Ws w = carve(a, (char*)a->workspace);
    HREQ(a->ws_bytes >= w.bytes, "workspace smaller than d8s_head_workspace()");
    hipStream_t st = (hipStream_t)stream;
    const int M = a->B * a->W;
    const int nblk = (a->D + TN - 1) / TN;
    k_head_valid<<<(M + NT - 1) / NT, NT, 0, st>>>(a->slot_mask, a->slot_of, w.valid, a->B, a->W, a->S);
    const dim3 gcd((M + TM - 1) / TM, (a->CD + TN - 1) / TN);
    {
        GemmP g{};
        g.M = M;
        g.W = a->W;
        g.slot_of = a->slot_of;
        g.slot_emb = a->slot_emb;
        // 1. h = (z + slot_emb) ctx_in^T + b + ctx_pos[w % per]
        g.A = a->z; g.Bw = a->ctx_in_w; g.bias = a->ctx_in_b; g.C = w.h;
        g.N = a->CD; g.K = a->D; g.ldc = a->CD; g.pos = a->ctx_pos; g.per = a->PER;
        k_head_gemm<PRO_SLOT, EPI_BIAS_POS><<<gcd, NT, 0, st>>>(g);
        // 2. qkv = LN1(h) in_proj^T + b
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.h; g.Bw = a->in_proj_w; g.bias = a->in_proj_b; g.C = w.qkv;
        g.N = 3 * a->CD; g.K = a->CD; g.ldc = 3 * a->CD; g.ln_w = a->ln1_w; g.ln_b = a->ln1_b;
        k_head_gemm<PRO_LN, EPI_BIAS><<<dim3((M + TM - 1) / TM, (3 * a->CD + TN - 1) / TN), NT, 0, st>>>(g);
        // 3. attention per (study, head)
        AttnP at{w.qkv, w.valid, w.att, a->W, a->CD, a->heads};
        k_head_attn<<<dim3(a->B, a->heads), NT, 0, st>>>(at);
        // 4. h1 = h + att out_proj^T + b
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.att; g.Bw = a->out_proj_w; g.bias = a->out_proj_b; g.C = w.h1;
        g.N = a->CD; g.K = a->CD; g.ldc = a->CD; g.R = w.h;
        k_head_gemm<PRO_NONE, EPI_BIAS_RES><<<gcd, NT, 0, st>>>(g);
        // 5. u = relu(LN2(h1) ff1^T + b)
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.h1; g.Bw = a->ff1_w; g.bias = a->ff1_b; g.C = w.u;
        g.N = a->FF; g.K = a->CD; g.ldc = a->FF; g.ln_w = a->ln2_w; g.ln_b = a->ln2_b;
        k_head_gemm<PRO_LN, EPI_BIAS_RELU><<<dim3((M + TM - 1) / TM, (a->FF + TN - 1) / TN), NT, 0, st>>>(g);
        // 6. h2 = h1 + u ff2^T + b
        g = GemmP{}; g.M = M; g.W = a->W;
        g.A = w.u; g.Bw = a->ff2_w; g.bias = a->ff2_b; g.C = w.h2;
        g.N = a->CD; g.K = a->FF; g.ldc = a->CD; g.R = w.h1;
        k_head_gemm<PRO_NONE, EPI_BIAS_RES><<<gcd, NT, 0, st>>>(g);
    }
    // 7. f2 = z + slot_emb + h2 ctx_out^T + b, partial dots with attn.weight and cls_w
    GemmP g{};
    g.M = M; g.W = a->W; g.slot_of = a->slot_of; g.slot_emb = a->slot_emb;
    g.N = a->D; g.z = a->z; g.tw = a->attn_w; g.cw = a->cls_w; g.part = w.part; g.T = a->T;
    g.A = w.h2; g.Bw = a->ctx_out_w; g.bias = a->ctx_out_b; g.K = a->CD;
    k_head_gemm<PRO_NONE, EPI_DOTS><<<dim3((M + TM - 1) / TM, nblk), NT, 0, st>>>(g);
    // 8. pooling
    PoolP pp{w.part, w.valid, a->attn_b, a->cls_b, a->logits, a->W, a->T, nblk};
    k_head_pool<<<a->B, NT, 0, st>>>(pp);
    return d8s_host_launched("d8s_head");
}
