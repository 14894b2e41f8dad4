// mlp_activation.h -- the activation step of the reference's MLP::forward
// (src/layers/mlp.cpp:270-292): after the gate and up GEMMs, SwiGLU
// (ActKind::Silu) or GeGLU (ActKind::GeluTanh) produces the [B, I] input of
// the down GEMM.  The GEMMs themselves are not part of this library.
#pragma once

#include "core/tensor.h"

namespace mini_infer {

// Activation selector, same enumerators as src/model/model_config.h:35-38.
enum class ActKind {
    Silu = 0,
    GeluTanh,
};

// out = act(gate) * up, elementwise; gate, up, out: fp16 of equal size on
// one GPU (out may be gate or up).  GeluTanh runs as one fused pass where
// the reference launches gelu_tanh then mul_inplace.
void apply_gated_activation(ActKind act, const Tensor& gate, const Tensor& up, Tensor& out);

}  // namespace mini_infer
