// train.hip - the elementwise, row and reduction kernels of the training
// step on gfx950 (the products go through launch_gemm, attention through
// attn_bwd.hip). Reference: gpt_forward with targets, gpt_backward and
// gpt_adamw (src/model.c:442-921) over the ops of src/ops.c:125-640.
//
// Every reduction here is deterministic: per-column sums over rows are
// formed as partial sums of fixed row chunks, then the chunks are summed in
// order by a second launch (no atomics), so repeated steps give the same
// bits.
#include "common.h"
#include "kernels.h"

namespace {

// ---------------------------------------------------------------- GELU

// out = gelu(in) over n4 float4 (the forward keeps the pre-activation for
// the backward, so GELU is not folded into the fc product here).
__global__ void __launch_bounds__(256) k_gelu_fwd(const f32x4* __restrict__ in,
                                                  f32x4* __restrict__ out, long n4) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const f32x4 v = in[i];
    out[i] = f32x4{gelu_tanh(v.x), gelu_tanh(v.y), gelu_tanh(v.z), gelu_tanh(v.w)};
}

// x[i] *= mask[i] ? scale : 0, over n4 groups of 4: dropout_fwd's scaling
// of the kept values and dropout_bwd's of the gradient (reference
// ops.c:603-625), the same product in both, with the mask drawn on the host.
__global__ void __launch_bounds__(256) k_dropout(f32x4* __restrict__ x,
                                                 const unsigned* __restrict__ mask, long n4,
                                                 float scale) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const unsigned m = mask[i];  // four mask bytes, element j in byte j
    f32x4 v = x[i];
    v.x *= (m & 0xffu) ? scale : 0.0f;
    v.y *= (m & 0xff00u) ? scale : 0.0f;
    v.z *= (m & 0xff0000u) ? scale : 0.0f;
    v.w *= (m & 0xff000000u) ? scale : 0.0f;
    x[i] = v;
}

// d gelu / dx of the tanh form (reference ops.c:347-355): 0.5 (1 + t) +
// 0.5 x (1 - t^2) u'(x), t = tanh(u), u = sqrt(2/pi) (x + 0.044715 x^3).
__device__ __forceinline__ float gelu_grad(float x) {
    const float k0 = 0.7978845608028654f, k1 = 0.044715f;
    const float u = k0 * (x + k1 * (x * x * x));
    const float t = tanhf(u);
    const float du = k0 * (1.0f + 3.0f * k1 * x * x);
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * du;
}

// d[i] = d[i] * gelu'(x[i]) (gelu_bwd, ops.c:382-422, into the buffer that
// held the gradient of the GELU output).
__global__ void __launch_bounds__(256) k_gelu_bwd(f32x4* __restrict__ d,
                                                  const f32x4* __restrict__ x, long n4) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const f32x4 g = d[i], v = x[i];
    d[i] = f32x4{g.x * gelu_grad(v.x), g.y * gelu_grad(v.y), g.z * gelu_grad(v.z),
                 g.w * gelu_grad(v.w)};
}

// ---------------------------------------------------------------- transpose

// dst[c * ldd + r] = src[r * lds + c] for r < rows, c < cols, and zero for
// the padding r in [rows, rows_p) or c in [cols, cols_p): the products of
// the backward take both operands K-contiguous, so the operand whose K is
// the row index (activations and gradients over B*T rows, the weights of
// dX = dY W) is transposed, with K padded to whole product steps. 64 x 64
// tiles through LDS (one padded column per row keeps the column reads
// conflict-free); reads along c and writes along r are both coalesced.
// With colpart set, the tile's column sums over its 64 rows (in row order)
// go to colpart[blockIdx.y][c]: the bias gradient's partial sums, formed
// while dY passes through anyway.
__global__ void __launch_bounds__(256) k_transpose(const float* __restrict__ src, long lds,
                                                   int rows, int cols, float* __restrict__ dst,
                                                   long ldd, int rows_p, int cols_p,
                                                   float* __restrict__ colpart) {
    __shared__ float t[64][65];
    __shared__ float cs[4][64];
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int r = r0 + 16 * ty + i, c = c0 + tx;
        t[16 * ty + i][tx] = (r < rows && c < cols) ? src[(long)r * lds + c] : 0.f;
    }
    __syncthreads();
    if (colpart) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) sum += t[16 * ty + i][tx];
        cs[ty][tx] = sum;
        __syncthreads();
        if (ty == 0 && c0 + tx < cols)
            colpart[(long)blockIdx.y * cols + c0 + tx] = ((cs[0][tx] + cs[1][tx]) + cs[2][tx]) + cs[3][tx];
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int c = c0 + ty + 4 * i, r = r0 + tx;
        if (c < cols_p && r < rows_p) dst[(long)c * ldd + r] = t[tx][ty + 4 * i];
    }
}

// ---------------------------------------------------------------- column sums

constexpr int CS_ROWS = 64;  // rows per partial column sum

// part[chunk][c] = sum of Y[r][c] over the chunk's CS_ROWS rows, in order
// (eight loads in flight per thread).
__global__ void __launch_bounds__(256) k_colsum_part(const float* __restrict__ Y, long ldy,
                                                     int rows, int cols,
                                                     float* __restrict__ part) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    const int r0 = blockIdx.y * CS_ROWS, r1 = min(rows, r0 + CS_ROWS);
    float s = 0.f;
    for (int r = r0; r < r1; r += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = Y[(long)min(r + j, r1 - 1) * ldy + c];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (r + j < r1) s += v[j];
    }
    part[(long)blockIdx.y * cols + c] = s;
}

// out[c] += sum over the nparts partials of column c: eight threads per
// column each sum a contiguous run of partials (eight loads in flight),
// then the eight run sums are added in run order.
constexpr int FIN_SPLIT = 8;
__global__ void __launch_bounds__(256) k_colsum_fin(const float* __restrict__ part, int nparts,
                                                    int cols, float* __restrict__ out) {
    __shared__ float rs[FIN_SPLIT][256 / FIN_SPLIT];
    const int cl = threadIdx.x % (256 / FIN_SPLIT), q = threadIdx.x / (256 / FIN_SPLIT);
    const int c = blockIdx.x * (256 / FIN_SPLIT) + cl;
    const int per = (nparts + FIN_SPLIT - 1) / FIN_SPLIT;
    const int p0 = q * per, p1 = min(nparts, p0 + per);
    float s = 0.f;
    if (c < cols)
        for (int p = p0; p < p1; p += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = part[(long)min(p + j, p1 - 1) * cols + c];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (p + j < p1) s += v[j];
        }
    rs[q][cl] = s;
    __syncthreads();
    if (q == 0 && c < cols) {
        float t = rs[0][cl];
#pragma unroll
        for (int k = 1; k < FIN_SPLIT; k++) t += rs[k][cl];
        out[c] += t;
    }
}

// ---------------------------------------------------------------- LayerNorm backward

constexpr int LNB_ROWS = 32;  // rows per workgroup (eight per wavefront)

// layernorm_bwd (ops.c:250-331) for LNB_ROWS rows per workgroup, one
// wavefront per row at a time (float4 columns lane + 64 j, NCH per lane):
// sum1 = mean(dn), sum2 = mean(dn * xhat) with dn = dout * w and xhat =
// (x - mean) * rstd, then dx += rstd * (dn - sum1 - xhat * sum2). The
// workgroup's share of dw (sum of dout * xhat) and db (sum of dout) is
// summed over its rows in order (each wavefront over its rows, then the
// four wavefronts in order through LDS) into part_dw / part_db [block][C].
template <int NCH>
__global__ void __launch_bounds__(256) k_ln_bwd(const float* __restrict__ dout,
                                                const float* __restrict__ x,
                                                const float* __restrict__ w,
                                                const float* __restrict__ mean,
                                                const float* __restrict__ rstd,
                                                float* __restrict__ dx, int rows, int C,
                                                float* __restrict__ part_dw,
                                                float* __restrict__ part_db) {
    __shared__ f32x4 red[2][4][64 * NCH];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int C4 = C >> 2;
    f32x4 wv[NCH], adw[NCH], adb[NCH];
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c4 = lane + 64 * j;
        wv[j] = ld4_or0((const f32x4*)w + min(c4, C4 - 1), c4 < C4);
        adw[j] = adb[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int rb = blockIdx.x * LNB_ROWS;
    for (int i = wave; i < LNB_ROWS; i += 4) {
        const int r = rb + i;
        if (r >= rows) break;
        const f32x4* dr = (const f32x4*)(dout + (long)r * C);
        const f32x4* xr = (const f32x4*)(x + (long)r * C);
        const float m = mean[r], rs = rstd[r];
        f32x4 dv[NCH], xh[NCH];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int c4 = lane + 64 * j;
            const bool ok = c4 < C4;
            dv[j] = ld4_or0(dr + min(c4, C4 - 1), ok);
            xh[j] = (ld4_or0(xr + min(c4, C4 - 1), ok) - m) * rs;
            const f32x4 dn = dv[j] * wv[j];
            const f32x4 p = dn * xh[j];
            s1 += (dn.x + dn.y) + (dn.z + dn.w);
            s2 += (p.x + p.y) + (p.z + p.w);
        }
        s1 = wave_sum_dpp(s1) / (float)C;
        s2 = wave_sum_dpp(s2) / (float)C;
        f32x4* dxr = (f32x4*)(dx + (long)r * C);
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int c4 = lane + 64 * j;
            if (c4 < C4) {
                const f32x4 dn = dv[j] * wv[j];
                dxr[c4] += rs * (dn - s1 - xh[j] * s2);
            }
            adw[j] += dv[j] * xh[j];
            adb[j] += dv[j];
        }
    }
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        red[0][wave][lane + 64 * j] = adw[j];
        red[1][wave][lane + 64 * j] = adb[j];
    }
    __syncthreads();
    for (int c4 = threadIdx.x; c4 < C4; c4 += 256) {
        const f32x4 sw = ((red[0][0][c4] + red[0][1][c4]) + red[0][2][c4]) + red[0][3][c4];
        const f32x4 sb = ((red[1][0][c4] + red[1][1][c4]) + red[1][2][c4]) + red[1][3][c4];
        ((f32x4*)(part_dw + (long)blockIdx.x * C))[c4] = sw;
        ((f32x4*)(part_db + (long)blockIdx.x * C))[c4] = sb;
    }
}

// ---------------------------------------------------------------- embedding backward

// g_wpe[t][c] += sum over b of dx[b][t][c], in b order (model.c:850-858).
__global__ void __launch_bounds__(256) k_wpe_bwd(const float* __restrict__ dx, int B, int T,
                                                 int C, float* __restrict__ g_wpe) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)T * C) return;
    float s = g_wpe[i];
    for (int b = 0; b < B; b++) s += dx[(long)b * T * C + i];
    g_wpe[i] = s;
}

// g_wte[tok] += dx rows of every position holding tok, in position order
// (model.c:859-866): one workgroup per distinct token u, whose positions
// are pos[start[u] .. start[u + 1]) (ascending).
__global__ void __launch_bounds__(256) k_wte_bwd(const float* __restrict__ dx, int C,
                                                 const int* __restrict__ uniq,
                                                 const int* __restrict__ start,
                                                 const int* __restrict__ pos,
                                                 float* __restrict__ g_wte) {
    const int u = blockIdx.x;
    const int tok = uniq[u], p0 = start[u], p1 = start[u + 1];
    float* g = g_wte + (long)tok * C;
    for (int c = threadIdx.x; c < C; c += 256) {
        float s = g[c];
        for (int p = p0; p < p1; p++) s += dx[(long)pos[p] * C + c];
        g[c] = s;
    }
}

// ---------------------------------------------------------------- gradient norm and AdamW

constexpr int SQ_BLOCK_ELEMS = 256 * 64;  // elements per partial sum of squares

// part[block] = sum of g^2 over the block's SQ_BLOCK_ELEMS elements, in
// double: each thread over its strided elements, then a fixed-order tree.
__global__ void __launch_bounds__(256) k_sumsq_part(const float* __restrict__ g, long n,
                                                    double* __restrict__ part) {
    __shared__ double red[256];
    const long base = (long)blockIdx.x * SQ_BLOCK_ELEMS;
    double s = 0.0;
    for (int k = 0; k < SQ_BLOCK_ELEMS / 256; k++) {
        const long i = base + k * 256 + threadIdx.x;
        if (i < n) s += (double)g[i] * (double)g[i];
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// norm[0] = sqrt(sum of the partials, in order); coef[0] = clip / norm when
// clip > 0 and norm > clip, else 1 (global_grad_norm / scale_grads,
// ops.c:631-640, as gpt_adamw applies them, model.c:893-900).
// One workgroup: thread i sums partials i, i + 256, .. in order, then a
// fixed-order tree.
__global__ void __launch_bounds__(256) k_norm_fin(const double* __restrict__ part, int nparts,
                                                  float clip, float* __restrict__ norm,
                                                  float* __restrict__ coef) {
    __shared__ double red[256];
    double s = 0.0;
    for (int p = threadIdx.x; p < nparts; p += 256) s += part[p];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float nv = (float)sqrt(red[0]);
        norm[0] = nv;
        coef[0] = (clip > 0.0f && nv > clip) ? clip / nv : 1.0f;
    }
}

// gpt_adamw's update (model.c:901-919) with the gradient scaled by *coef
// first (and stored back, as scale_grads does): decoupled weight decay on
// the elements whose decay byte is set.
__global__ void __launch_bounds__(256) k_adamw(float* __restrict__ p, float* __restrict__ g,
                                               float* __restrict__ m, float* __restrict__ v,
                                               const unsigned char* __restrict__ decay, long n,
                                               const float* __restrict__ coef, float lr,
                                               float beta1, float beta2, float eps, float wd,
                                               float bc1, float bc2) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float s = coef[0];
    float gi = g[i];
    if (s != 1.0f) {
        gi *= s;
        g[i] = gi;
    }
    const float mi = beta1 * m[i] + (1.0f - beta1) * gi;
    const float vi = beta2 * v[i] + (1.0f - beta2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const float mh = mi / bc1, vh = vi / bc2;
    const float ewd = decay[i] ? wd : 0.0f;
    p[i] = p[i] * (1.0f - lr * ewd) - lr * mh / (sqrtf(vh) + eps);
}

}  // namespace

// ---------------------------------------------------------------- launchers

hipError_t launch_gelu_fwd(const float* in, float* out, long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n & 3) return hipErrorInvalidValue;
    const long n4 = n >> 2;
    k_gelu_fwd<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>((const f32x4*)in, (f32x4*)out, n4);
    return hipGetLastError();
}

hipError_t launch_dropout(float* x, const unsigned char* mask, long n, float scale,
                          hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n & 3) return hipErrorInvalidValue;
    const long n4 = n >> 2;
    k_dropout<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>((f32x4*)x, (const unsigned*)mask, n4,
                                                           scale);
    return hipGetLastError();
}

hipError_t launch_gelu_bwd(float* d, const float* x, long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n & 3) return hipErrorInvalidValue;
    const long n4 = n >> 2;
    k_gelu_bwd<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>((f32x4*)d, (const f32x4*)x, n4);
    return hipGetLastError();
}

hipError_t launch_transpose(const float* src, long lds, int rows, int cols, float* dst, long ldd,
                            int rows_p, int cols_p, hipStream_t s) {
    if (rows_p <= 0 || cols_p <= 0) return hipSuccess;
    if (rows_p < rows || cols_p < cols || ldd < rows_p) return hipErrorInvalidValue;
    dim3 grid((cols_p + 63) / 64, (rows_p + 63) / 64);
    k_transpose<<<grid, 256, 0, s>>>(src, lds, rows, cols, dst, ldd, rows_p, cols_p, nullptr);
    return hipGetLastError();
}

long transpose_colsum_floats(int rows, int cols) { return (long)((rows + 63) / 64) * cols; }

hipError_t launch_transpose_colsum(const float* src, long lds, int rows, int cols, float* dst,
                                   long ldd, int rows_p, int cols_p, float* part, float* out,
                                   hipStream_t s) {
    if (rows_p <= 0 || cols_p <= 0) return hipSuccess;
    if (rows_p < rows || cols_p < cols || ldd < rows_p) return hipErrorInvalidValue;
    dim3 grid((cols_p + 63) / 64, (rows_p + 63) / 64);
    k_transpose<<<grid, 256, 0, s>>>(src, lds, rows, cols, dst, ldd, rows_p, cols_p, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nparts = (rows_p + 63) / 64;
    k_colsum_fin<<<(cols + 31) / 32, 256, 0, s>>>(part, nparts, cols, out);
    return hipGetLastError();
}

long colsum_part_floats(int rows, int cols) {
    return (long)((rows + CS_ROWS - 1) / CS_ROWS) * cols;
}

hipError_t launch_colsum_add(const float* Y, long ldy, int rows, int cols, float* part,
                             float* out, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const int nparts = (rows + CS_ROWS - 1) / CS_ROWS;
    k_colsum_part<<<dim3((cols + 255) / 256, nparts), 256, 0, s>>>(Y, ldy, rows, cols, part);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_colsum_fin<<<(cols + 31) / 32, 256, 0, s>>>(part, nparts, cols, out);
    return hipGetLastError();
}

long ln_bwd_part_floats(int rows, int C) {
    return 2L * ((rows + LNB_ROWS - 1) / LNB_ROWS) * C;
}

hipError_t launch_layernorm_bwd(const float* dout, const float* x, const float* w,
                                const float* mean, const float* rstd, float* dx, float* dw,
                                float* db, int rows, int C, float* part, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (C & 3) return hipErrorInvalidValue;
    const int nb = (rows + LNB_ROWS - 1) / LNB_ROWS;
    float* pdw = part;
    float* pdb = part + (long)nb * C;
    const int nch = (C / 4 + 63) / 64;
#define LNB(N) k_ln_bwd<N><<<nb, 256, 0, s>>>(dout, x, w, mean, rstd, dx, rows, C, pdw, pdb)
    if (nch <= 1) LNB(1);
    else if (nch <= 2) LNB(2);
    else if (nch <= 3) LNB(3);
    else if (nch <= 4) LNB(4);
    else if (nch <= 8) LNB(8);
    else return hipErrorInvalidValue;
#undef LNB
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_colsum_fin<<<(C + 31) / 32, 256, 0, s>>>(pdw, nb, C, dw);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_colsum_fin<<<(C + 31) / 32, 256, 0, s>>>(pdb, nb, C, db);
    return hipGetLastError();
}

hipError_t launch_embed_bwd(const float* dx, int B, int T, int C, float* g_wpe, float* g_wte,
                            const int* uniq, const int* start, const int* pos, int nuniq,
                            hipStream_t s) {
    const long n = (long)T * C;
    if (n > 0) {
        k_wpe_bwd<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(dx, B, T, C, g_wpe);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (nuniq <= 0) return hipSuccess;
    k_wte_bwd<<<nuniq, 256, 0, s>>>(dx, C, uniq, start, pos, g_wte);
    return hipGetLastError();
}

int grad_norm_parts(long n) { return (int)((n + SQ_BLOCK_ELEMS - 1) / SQ_BLOCK_ELEMS); }

hipError_t launch_adamw(float* p, float* g, float* m, float* v, const unsigned char* decay,
                        long n, double* part, float* norm, float* coef, float lr, float beta1,
                        float beta2, float eps, float wd, float clip, float bc1, float bc2,
                        hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int np = grad_norm_parts(n);
    k_sumsq_part<<<np, 256, 0, s>>>(g, n, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_norm_fin<<<1, 256, 0, s>>>(part, np, clip, norm, coef);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_adamw<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(p, g, m, v, decay, n, coef, lr, beta1,
                                                        beta2, eps, wd, bc1, bc2);
    return hipGetLastError();
}
