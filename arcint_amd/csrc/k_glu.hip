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

// grid: x over the rows in 256-row blocks, y over the columns of all batches (col = c + N b):
// no division per element
template <int OP>
__global__ __launch_bounds__(256) void k_glu(GluArgs a, uint32_t col0) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m >= a.M) return;
    const uint32_t col = col0 + blockIdx.y, c = col % (uint32_t)a.N, b = col / (uint32_t)a.N;
    const uint32_t i2 = b % (uint32_t)a.ne12, i3 = b / (uint32_t)a.ne12;
    const int64_t i = (int64_t)col * a.M + m;
    const float x = a.gate[i], g = a.up[i];
    // REGLU keeps ggml's form (x > 0 ? x g : 0); the others act(x) * g
    const float y = OP == QMM_GLU_REGLU ? (x > 0.0f ? x * g : 0.0f) : glu_act(OP, x) * g;
    a.dst[m + (int64_t)c * a.d_nb1 + (int64_t)i2 * a.d_nb2 + (int64_t)i3 * a.d_nb3] = y;
}

}  // namespace

hipError_t launch_glu(int op, const GluArgs & a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0 || a.nb <= 0) return hipSuccess;
    const int64_t cols = a.N * a.nb;
    if ((a.M + 255) / 256 > 0x7fffffff || cols > 0xffffffffll) return hipErrorInvalidValue;
    for (int64_t c0 = 0; c0 < cols; c0 += 65535) {                 // grid y: up to 65535 columns a launch
        const dim3 g((unsigned)((a.M + 255) / 256), (unsigned)std::min<int64_t>(65535, cols - c0)), b(256);
        switch (op) {
            case QMM_GLU_REGLU:       k_glu<QMM_GLU_REGLU><<<g, b, 0, s>>>(a, (uint32_t)c0); break;
            case QMM_GLU_GEGLU:       k_glu<QMM_GLU_GEGLU><<<g, b, 0, s>>>(a, (uint32_t)c0); break;
            case QMM_GLU_SWIGLU:      k_glu<QMM_GLU_SWIGLU><<<g, b, 0, s>>>(a, (uint32_t)c0); break;
            case QMM_GLU_GEGLU_ERF:   k_glu<QMM_GLU_GEGLU_ERF><<<g, b, 0, s>>>(a, (uint32_t)c0); break;
            case QMM_GLU_GEGLU_QUICK: k_glu<QMM_GLU_GEGLU_QUICK><<<g, b, 0, s>>>(a, (uint32_t)c0); break;
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

}  // namespace qmm
