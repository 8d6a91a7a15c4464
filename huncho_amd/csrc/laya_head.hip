// laya_head.hip - the elementwise kernels of the typed Laya decision head (LayaHead,
// crates/huncho-backend/src/candle.rs:500-694) on gfx950. The head's GEMMs run on hipBLASLt,
// its attention on bidir_attn (bert.hip) and its LayerNorms on layer_norm (bert.hip).
//
//   type_add<T>     z = T(h + type_emb[qtype of the row's sequence])         (candle.rs:658-659)
//   bias_act<T,A>   y = T(act(T(x + b)))  or  y = T(r + T(act(T(x + b))))   (the bias of each
//                   Linear, the ReLU of the FFN / the erf GELU of the scorer, the residual adds)
//   gather_rows<T>  the rows at the readout positions                          (candle.rs:675-680)
//   score_dot<T>    the scorer's last Linear(a -> 1): T(T(y . w) + b) per position
// Each result is rounded to the activation dtype where the reference stores a tensor of it.
#include "common.hpp"
#include "kernel_args.hpp"

namespace hk {
namespace laya {

template <typename T> struct V8 { typedef typename Mma16<T>::v8 type; };
template <> struct V8<float> { typedef float __attribute__((ext_vector_type(8))) type; };

template <typename T> __device__ __forceinline__ float rnd(float x) { return to_f(from_f<T>(x)); }

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

__device__ __forceinline__ int seq_of(const int* cu, int n, int t) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// one thread per 8 consecutive elements of a row (width % 8 == 0, 16-byte aligned rows)
template <typename T>
__global__ __launch_bounds__(256) void type_add(LayaTypeArgs a) {
    typedef typename V8<T>::type v8;
    const int per_row = a.width / 8;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)a.rows * per_row) return;
    const int r = (int)(i / per_row), c = (int)(i % per_row) * 8;
    const int s = seq_of(a.cu, a.n_seqs, r);
    const float* te = a.type_emb + (long)a.qtype[s] * a.width + c;
    const v8 x = *(const v8*)((const T*)a.x + (long)r * a.x_tok + c);
    v8 y;
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = from_f<T>(to_f(x[e]) + te[e]);
    *(v8*)((T*)a.y + (long)r * a.y_tok + c) = y;
}

template <typename T, int ACT>
__global__ __launch_bounds__(256) void bias_act(LayaBiasArgs a) {
    typedef typename V8<T>::type v8;
    const int per_row = a.width / 8;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)a.rows * per_row) return;
    const int r = (int)(i / per_row), c = (int)(i % per_row) * 8;
    const v8 x = *(const v8*)((const T*)a.x + (long)r * a.x_tok + c);
    v8 res;
    if (a.res) res = *(const v8*)((const T*)a.res + (long)r * a.res_tok + c);
    v8 y;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float t = rnd<T>(to_f(x[e]) + a.b[c + e]);
        if (ACT == 1) t = fmaxf(t, 0.0f);
        if (ACT == 2) t = rnd<T>(gelu_erf(t));
        y[e] = a.res ? from_f<T>(to_f(res[e]) + t) : from_f<T>(t);
    }
    *(v8*)((T*)a.y + (long)r * a.y_tok + c) = y;
}

// position p of the flattened readout list -> its row: cu[s] + positions[p], s the sequence
// whose position range holds p
template <typename T>
__global__ __launch_bounds__(256) void gather_rows(LayaGatherArgs a) {
    typedef typename V8<T>::type v8;
    const int per_row = a.width / 8;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)a.n_positions * per_row) return;
    const int p = (int)(i / per_row), c = (int)(i % per_row) * 8;
    const int s = seq_of(a.cu_positions, a.n_seqs, p);
    const long row = (long)a.cu[s] + a.positions[p];
    *(v8*)((T*)a.y + (long)p * a.width + c) = *(const v8*)((const T*)a.x + row * a.x_tok + c);
}

// one wave per position: fp32 dot over the (zero-padded) scorer width
template <typename T>
__global__ __launch_bounds__(256) void score_dot(LayaScoreArgs a) {
    const int p = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (p >= a.n_positions) return;
    const T* y = (const T*)a.y + (long)p * a.width;
    float s = 0.0f;
    for (int c = lane; c < a.width; c += 64) s += to_f(y[c]) * a.w[c];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) a.out[p] = rnd<T>(rnd<T>(s) + a.b);
}

}  // namespace laya
}  // namespace hk

#define HK_LAYA_DISPATCH(dtype, KERNEL, grid, stream, args)                                             \
    do {                                                                                                \
        if ((dtype) == hk::DT_BF16) hipLaunchKernelGGL(hk::laya::KERNEL<hk::bf16>, grid, dim3(256), 0, stream, args); \
        else if ((dtype) == hk::DT_F16) hipLaunchKernelGGL(hk::laya::KERNEL<hk::f16>, grid, dim3(256), 0, stream, args); \
        else hipLaunchKernelGGL(hk::laya::KERNEL<float>, grid, dim3(256), 0, stream, args);            \
    } while (0)

static dim3 grid_for(long items) { return dim3((unsigned)((items + 255) / 256)); }

extern "C" int hk_launch_laya_type_add(int dtype, const hk::LayaTypeArgs* a, hipStream_t stream) {
    if (a->rows == 0) return HK_OK;
    HK_LAYA_DISPATCH(dtype, type_add, grid_for((long)a->rows * (a->width / 8)), stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

extern "C" int hk_launch_laya_bias_act(int dtype, int act, const hk::LayaBiasArgs* a, hipStream_t stream) {
    if (a->rows == 0) return HK_OK;
    const dim3 g = grid_for((long)a->rows * (a->width / 8));
    if (act == 1) {
        if (dtype == hk::DT_BF16) hipLaunchKernelGGL((hk::laya::bias_act<hk::bf16, 1>), g, dim3(256), 0, stream, *a);
        else if (dtype == hk::DT_F16) hipLaunchKernelGGL((hk::laya::bias_act<hk::f16, 1>), g, dim3(256), 0, stream, *a);
        else hipLaunchKernelGGL((hk::laya::bias_act<float, 1>), g, dim3(256), 0, stream, *a);
    } else if (act == 2) {
        if (dtype == hk::DT_BF16) hipLaunchKernelGGL((hk::laya::bias_act<hk::bf16, 2>), g, dim3(256), 0, stream, *a);
        else if (dtype == hk::DT_F16) hipLaunchKernelGGL((hk::laya::bias_act<hk::f16, 2>), g, dim3(256), 0, stream, *a);
        else hipLaunchKernelGGL((hk::laya::bias_act<float, 2>), g, dim3(256), 0, stream, *a);
    } else {
        if (dtype == hk::DT_BF16) hipLaunchKernelGGL((hk::laya::bias_act<hk::bf16, 0>), g, dim3(256), 0, stream, *a);
        else if (dtype == hk::DT_F16) hipLaunchKernelGGL((hk::laya::bias_act<hk::f16, 0>), g, dim3(256), 0, stream, *a);
        else hipLaunchKernelGGL((hk::laya::bias_act<float, 0>), g, dim3(256), 0, stream, *a);
    }
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

extern "C" int hk_launch_laya_gather(int dtype, const hk::LayaGatherArgs* a, hipStream_t stream) {
    if (a->n_positions == 0) return HK_OK;
    HK_LAYA_DISPATCH(dtype, gather_rows, grid_for((long)a->n_positions * (a->width / 8)), stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}

extern "C" int hk_launch_laya_score(int dtype, const hk::LayaScoreArgs* a, hipStream_t stream) {
    if (a->n_positions == 0) return HK_OK;
    HK_LAYA_DISPATCH(dtype, score_dot, dim3((unsigned)((a->n_positions + 3) / 4)), stream, *a);
    return hipGetLastError() == hipSuccess ? HK_OK : HK_ERR_DEVICE;
}
