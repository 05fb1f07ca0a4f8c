// rowops.hip - bandwidth-bound row kernels: token+position embedding,
// LayerNorm and row gather.
//
// All are HBM-bound. Each row of C floats is owned by one wavefront and
// moved with 16-byte loads; reductions stay inside the wavefront (butterfly
// shuffles), so no LDS or block barrier is needed.
#include "common.h"
#include "kernels.h"

// x[i, :] = wte[tok[i], :] + wpe[pos0 + i % T, :]   (reference fast.c:245-254)
// One thread per float4. pos0 comes from *pos_dev when pos_dev is set, so a
// captured decode step can advance the position on the device. Token ids
// outside [0, V) are clamped and reported through *err. With hist set, the
// token of row i is also recorded at hist[i * hist_stride + position].
__global__ void __launch_bounds__(256) k_embed(const int* __restrict__ tok,
                                               const float* __restrict__ wte,
                                               const float* __restrict__ wpe, float* __restrict__ x,
                                               long rows, int T, int C, int V, int pos0,
                                               const int* __restrict__ pos_dev, int* __restrict__ err,
                                               int* __restrict__ hist, long hist_stride) {
    const int c4 = C >> 2;
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * c4) return;
    long r = i / c4;
    int c = (int)(i - r * c4) * 4;
    int t = (int)(r % T) + (pos_dev ? *pos_dev : pos0);
    int id = tok[r];
    if (id < 0 || id >= V) {
        if (err) atomicOr(err, 1);
        id = id < 0 ? 0 : V - 1;
    }
    if (hist && c == 0) hist[r * hist_stride + t] = tok[r];
    f32x4 a = *(const f32x4*)(wte + (long)id * C + c);
    f32x4 b = *(const f32x4*)(wpe + (long)t * C + c);
    *(f32x4*)(x + r * C + c) = a + b;
}

// LayerNorm of one row per wavefront (reference ops.c:191-248): mean, biased
// variance of (x - mean), rstd = 1/sqrtf(var + 1e-5), out = (x-m)*rstd*w + b;
// with mean_out / rstd_out set, also each row's mean and rstd (the training
// forward keeps them for the backward, as layernorm_fwd does).
// NCH = float4 chunks per lane, so C <= 256 * NCH. Rows are read at stride
// in_stride and written at stride out_stride (floats), which lets the final
// LayerNorm of the last-position pass gather rows b*T + T-1.
template <int NCH>
__global__ void __launch_bounds__(256) k_layernorm(const float* __restrict__ x, long in_stride,
                                                   const float* __restrict__ w,
                                                   const float* __restrict__ b, float* __restrict__ out,
                                                   long out_stride, int rows, int C,
                                                   float* __restrict__ mean_out,
                                                   float* __restrict__ rstd_out) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (long)row * in_stride;
    // gain and bias are loaded with the row, not after the reductions
    f32x4 v[NCH], wv[NCH], bv[NCH];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int c = (lane + j * 64) * 4;
        const int cc = min(c, C - 4);
        v[j] = ld4_or0((const f32x4*)(xr + cc), c < C);
        wv[j] = ld4_or0((const f32x4*)(w + cc), c < C);
        bv[j] = ld4_or0((const f32x4*)(b + cc), c < C);
        s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    }
    const float m = wave_sum(s) / (float)C;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        int c = (lane + j * 64) * 4;
        if (c < C) {
            f32x4 d = v[j] - m;
            q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
    }
    const float rs = 1.0f / sqrtf(wave_sum(q) / (float)C + 1e-5f);
    if (mean_out && lane == 0) {
        mean_out[row] = m;
        rstd_out[row] = rs;
    }
    float* orow = out + (long)row * out_stride;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        int c = (lane + j * 64) * 4;
        if (c < C) *(f32x4*)(orow + c) = (v[j] - m) * rs * wv[j] + bv[j];
    }
}

// dst[r, :] = src[r * src_stride + src_off, :] for r < rows (C floats each).
__global__ void __launch_bounds__(256) k_gather_rows(const float* __restrict__ src, long src_stride,
                                                     float* __restrict__ dst, int rows, int C) {
    const int c4 = C >> 2;
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)rows * c4) return;
    int r = (int)(i / c4);
    int c = (int)(i - (long)r * c4) * 4;
    *(f32x4*)(dst + (long)r * C + c) = *(const f32x4*)(src + (long)r * src_stride + c);
}

// ---------------------------------------------------------------- launchers

hipError_t launch_embed(const int* tok, const float* wte, const float* wpe, float* x, long rows,
                        int T, int C, int V, int pos0, const int* pos_dev, int* err,
                        int* hist, long hist_stride, hipStream_t s) {
    long n = rows * (C / 4);
    if (n == 0) return hipSuccess;
    k_embed<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(tok, wte, wpe, x, rows, T, C, V, pos0,
                                                         pos_dev, err, hist, hist_stride);
    return hipGetLastError();
}

hipError_t launch_layernorm(const float* x, long in_stride, const float* w, const float* b,
                            float* out, long out_stride, int rows, int C, hipStream_t s,
                            float* mean, float* rstd) {
    if (rows == 0) return hipSuccess;
    if (!mean != !rstd) return hipErrorInvalidValue;
    dim3 grid((rows + 3) / 4), block(256);
    int nch = (C + 255) / 256;
    if (nch <= 1)
        k_layernorm<1><<<grid, block, 0, s>>>(x, in_stride, w, b, out, out_stride, rows, C, mean, rstd);
    else if (nch <= 2)
        k_layernorm<2><<<grid, block, 0, s>>>(x, in_stride, w, b, out, out_stride, rows, C, mean, rstd);
    else if (nch <= 3)
        k_layernorm<3><<<grid, block, 0, s>>>(x, in_stride, w, b, out, out_stride, rows, C, mean, rstd);
    else if (nch <= 4)
        k_layernorm<4><<<grid, block, 0, s>>>(x, in_stride, w, b, out, out_stride, rows, C, mean, rstd);
    else if (nch <= 8)
        k_layernorm<8><<<grid, block, 0, s>>>(x, in_stride, w, b, out, out_stride, rows, C, mean, rstd);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float* src, long src_stride, float* dst, int rows, int C,
                              hipStream_t s) {
    long n = (long)rows * (C / 4);
    if (n == 0) return hipSuccess;
    k_gather_rows<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(src, src_stride, dst, rows, C);
    return hipGetLastError();
}
