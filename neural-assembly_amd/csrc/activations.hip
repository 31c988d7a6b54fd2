// activations.hip -- the ten tensor-level activations plus sigmoid.
//
// Formulas are those of activations_c.c:124-158 (and node_sigmoid,
// activations.asm:352-413), evaluated in double for both dtypes and rounded
// once to float for f32 tensors (activations_c.c:71-77), with the same
// operation order and no FMA contraction.  exp/log/tanh are the ROCm device
// library's double routines; the reference uses glibc's, so transcendental
// results agree to the last few double ulps, not bit for bit.
#include <cmath>

#include "ew_impl.hpp"

namespace nh {

constexpr double kGelu = 0.7978845608028654;
constexpr double kSeluL = 1.0507009873554804934193349852946;
constexpr double kSeluA = 1.6732632423543772848170429916717;

struct ATanh { NH_DEV double f(double x) const { return tanh(x); } };
struct AGelu { NH_DEV double f(double x) const { return 0.5 * x * (1.0 + tanh(kGelu * (x + 0.044715 * x * x * x))); } };
struct ALeaky { double alpha; NH_DEV double f(double x) const { return x >= 0 ? x : alpha * x; } };
struct AElu { double alpha; NH_DEV double f(double x) const { return x > 0 ? x : alpha * (exp(x) - 1.0); } };
struct ASelu { NH_DEV double f(double x) const { return x > 0 ? kSeluL * x : kSeluL * kSeluA * (exp(x) - 1.0); } };
struct ASwish { NH_DEV double f(double x) const { return x / (1.0 + exp(-x)); } };
struct AMish { NH_DEV double f(double x) const { return x * tanh(log(1.0 + exp(x))); } };
struct AHardswish { NH_DEV double f(double x) const { return x <= -3.0 ? 0.0 : (x >= 3.0 ? x : x * (x + 3.0) / 6.0); } };
struct ASoftplus { NH_DEV double f(double x) const { return log(1.0 + exp(x)); } };
struct AHardtanh { NH_DEV double f(double x) const { return x < -1.0 ? -1.0 : (x > 1.0 ? 1.0 : x); } };
struct ASigmoid { NH_DEV double f(double x) const { return 1.0 / (1.0 + exp(x * -1.0)); } };

template <class A>
struct ActFn {
    A a;
    NH_DEV float operator()(float x) const { return float(a.f(double(x))); }
    NH_DEV double operator()(double x) const { return a.f(x); }
};

template <class A>
static int act(void *out, const void *in, A a = A{})
{
    if (!out || !in) return set_error(NEURAL_ERR_NULL_POINTER);
    ActFn<A> f{a};
    return run_unary(static_cast<NeuralTensor *>(out), static_cast<const NeuralTensor *>(in), f, f);
}

}  // namespace nh

using namespace nh;

extern "C" {

int act_tanh(void *out, const void *in) { return act<ATanh>(out, in); }
int act_gelu(void *out, const void *in) { return act<AGelu>(out, in); }
int act_leaky_relu(void *out, const void *in, double alpha) { return act<ALeaky>(out, in, ALeaky{alpha}); }
int act_elu(void *out, const void *in, double alpha) { return act<AElu>(out, in, AElu{alpha}); }
int act_selu(void *out, const void *in) { return act<ASelu>(out, in); }
int act_swish(void *out, const void *in) { return act<ASwish>(out, in); }
int act_mish(void *out, const void *in) { return act<AMish>(out, in); }
int act_hardswish(void *out, const void *in) { return act<AHardswish>(out, in); }
int act_softplus(void *out, const void *in) { return act<ASoftplus>(out, in); }
int act_hardtanh(void *out, const void *in) { return act<AHardtanh>(out, in); }

// Tensor-typed aliases of the header's neural_* activations
// (neural_api.h:387-486).
int neural_sigmoid(NeuralTensor *out, const NeuralTensor *in) { return act<ASigmoid>(out, in); }
int neural_tanh(NeuralTensor *out, const NeuralTensor *in) { return act<ATanh>(out, in); }
int neural_gelu(NeuralTensor *out, const NeuralTensor *in) { return act<AGelu>(out, in); }
int neural_leaky_relu(NeuralTensor *out, const NeuralTensor *in, double alpha) { return act<ALeaky>(out, in, ALeaky{alpha}); }
int neural_elu(NeuralTensor *out, const NeuralTensor *in, double alpha) { return act<AElu>(out, in, AElu{alpha}); }
int neural_selu(NeuralTensor *out, const NeuralTensor *in) { return act<ASelu>(out, in); }
int neural_swish(NeuralTensor *out, const NeuralTensor *in) { return act<ASwish>(out, in); }
int neural_mish(NeuralTensor *out, const NeuralTensor *in) { return act<AMish>(out, in); }
int neural_hardswish(NeuralTensor *out, const NeuralTensor *in) { return act<AHardswish>(out, in); }
int neural_softplus(NeuralTensor *out, const NeuralTensor *in) { return act<ASoftplus>(out, in); }
int neural_hardtanh(NeuralTensor *out, const NeuralTensor *in) { return act<AHardtanh>(out, in); }

}  // extern "C"
