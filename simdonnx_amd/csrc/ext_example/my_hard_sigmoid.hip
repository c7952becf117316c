// A consumer extension operator's kernel, shipped in its own code object: the HIP counterpart of
// the MyHardSigmoid test op's "hsig" dispatch (tests/Sdcb.SimdOnnx.Tests/Api/ExtensionTests.cs:37-44).
// It is NOT embedded in libsoxbackend.so: the build writes it to _build/ext/my_hard_sigmoid.hsaco,
// the owner loads it with sox_backend_load_module (the reference's ShaderResources.Open of an
// extension assembly's embedded shader) and its emitter dispatches it with sox_graph_dispatch.
//
// Kernarg block = the dispatch's two binds (8-byte device addresses, in order) followed by the
// params bytes: count, alpha, beta (the reference's PcOfF([count], alpha, beta)).
#include <hip/hip_runtime.h>
#include <stdint.h>

struct my_hsig_args {
    const void* x;
    void* y;
    uint32_t count;
    float alpha, beta;
};

__device__ __forceinline__ float my_hsig(float v, float alpha, float beta) {
    return fminf(fmaxf(v * alpha + beta, 0.0f), 1.0f);
}

// fp16 / bf16 graphs store activations as 16-bit floats; the math is fp32 (the reference GPU contract)
extern "C" __global__ void __launch_bounds__(256) my_hsig_f16(my_hsig_args a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.count) return;
    const _Float16 v = ((const _Float16*)a.x)[i];
    ((_Float16*)a.y)[i] = (_Float16)my_hsig((float)v, a.alpha, a.beta);
}

extern "C" __global__ void __launch_bounds__(256) my_hsig_bf16(my_hsig_args a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.count) return;
    const __bf16 v = ((const __bf16*)a.x)[i];
    ((__bf16*)a.y)[i] = (__bf16)my_hsig((float)v, a.alpha, a.beta);
}

extern "C" __global__ void __launch_bounds__(256) my_hsig_f32(my_hsig_args a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.count) return;
    ((float*)a.y)[i] = my_hsig(((const float*)a.x)[i], a.alpha, a.beta);
}
