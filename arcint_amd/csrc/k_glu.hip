// k_glu.hip - the GLU of a gate/up pair on gfx950: dst = act(gate) * up, elementwise.
//
// Role of ggml's GGML_OP_GLU in its split form (two tensors), as the reference runs it after
// its fused gate+up GEMV (kernel_swiglu / kernel_geglu / ... of glu.cl, whose loops
// P01:1350-1470 reshapes).  The activations are ggml's scalar definitions (ggml-cpu vec.h):
//   REGLU        x > 0 ? x g : 0
//   GEGLU        0.5 x (1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2))) g
//   SWIGLU       x / (1 + exp(-x)) g
//   GEGLU_ERF    0.5 x (1 + erf(x / sqrt(2))) g
//   GEGLU_QUICK  x / (1 + exp(-1.702 x)) g
// computed in fp32 with the device library's expf / tanhf / erff.  gate and up are the GEMV's
// scratch [batch][N][M]; dst is written through its strides.
#include "qmm_device.h"

namespace qmm {
namespace {

#pragma clang fp contract(off)

__device__ __forceinline__ float glu_act(int op, float x) {
    switch (op) {
        case QMM_GLU_REGLU: return x > 0.0f ? x : 0.0f;
        case QMM_GLU_GEGLU: {
            const float k0 = 0.79788456080286535587989211986876f, k1 = 0.044715f;
            return 0.5f * x * (1.0f + tanhf(k0 * x * (1.0f + k1 * x * x)));
        }
        case QMM_GLU_SWIGLU: return x / (1.0f + expf(-x));
        case QMM_GLU_GEGLU_ERF: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440084436210484f));
        case QMM_GLU_GEGLU_QUICK: return x * (1.0f / (1.0f + expf(-1.702f * x)));
        default: return 0.0f;
    }
}

template <int OP>
__global__ __launch_bounds__(256) void k_glu(GluArgs a) {
    const int64_t n = a.M * a.N * a.nb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = i % a.M, col = i / a.M, c = col % a.N, b = col / a.N;
        const int64_t i2 = b % a.ne12, i3 = b / a.ne12;
        const float x = a.gate[i], g = a.up[i];
        // REGLU keeps ggml's form (x > 0 ? x g : 0); the others act(x) * g
        const float y = OP == QMM_GLU_REGLU ? (x > 0.0f ? x * g : 0.0f) : glu_act(OP, x) * g;
        a.dst[m + c * a.d_nb1 + i2 * a.d_nb2 + i3 * a.d_nb3] = y;
    }
}

}  // namespace

hipError_t launch_glu(int op, const GluArgs & a, hipStream_t s) {
    const int64_t n = a.M * a.N * a.nb;
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    const dim3 g((unsigned)blocks), b(256);
    switch (op) {
        case QMM_GLU_REGLU:       k_glu<QMM_GLU_REGLU><<<g, b, 0, s>>>(a); break;
        case QMM_GLU_GEGLU:       k_glu<QMM_GLU_GEGLU><<<g, b, 0, s>>>(a); break;
        case QMM_GLU_SWIGLU:      k_glu<QMM_GLU_SWIGLU><<<g, b, 0, s>>>(a); break;
        case QMM_GLU_GEGLU_ERF:   k_glu<QMM_GLU_GEGLU_ERF><<<g, b, 0, s>>>(a); break;
        case QMM_GLU_GEGLU_QUICK: k_glu<QMM_GLU_GEGLU_QUICK><<<g, b, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qmm
