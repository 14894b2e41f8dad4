// mlp_activation.cpp -- gated activation dispatch (reference: src/layers/mlp.cpp:270-292).
#include "layers/mlp_activation.h"

#include <stdexcept>

#include "kernels/gelu_kernel.h"
#include "kernels/swiglu_kernel.h"

namespace mini_infer {

void apply_gated_activation(ActKind act, const Tensor& gate, const Tensor& up, Tensor& out) {
    for (const Tensor* t : {&gate, &up, static_cast<const Tensor*>(&out)}) {
        if (t->dtype() != DType::FP16)
            throw std::runtime_error("apply_gated_activation: only FP16 supported");
        if (!t->device().is_cuda())
            throw std::runtime_error("apply_gated_activation: tensors must be on the GPU");
        if (!t->is_contiguous())
            throw std::runtime_error("apply_gated_activation: only contiguous tensors supported");
    }
    if (gate.numel() != up.numel() || out.numel() != gate.numel())
        throw std::runtime_error("apply_gated_activation: size mismatch");
    if (gate.device().index != up.device().index || out.device().index != gate.device().index)
        throw std::runtime_error("apply_gated_activation: device mismatch");
    const int64_t n = gate.numel();
    if (act == ActKind::Silu) {
        if (n > 2147483647) throw std::runtime_error("apply_gated_activation: n exceeds int range");
        kernels::launch_swiglu(static_cast<const __half*>(gate.data()),
                               static_cast<const __half*>(up.data()),
                               static_cast<__half*>(out.data()), static_cast<int>(n), 0);
    } else {
        kernels::launch_geglu(static_cast<const __half*>(gate.data()),
                              static_cast<const __half*>(up.data()),
                              static_cast<__half*>(out.data()), n, 0);
    }
}

}  // namespace mini_infer
