// torch ops of namespace vkwr_sampling (module _sampling_C): the reference's
// three sampling ops with byte-identical schemas (reference
// csrc/sampling/torch_bindings.cpp:36-48) and the argument handling of its
// host functions (csrc/sampling/sampling.cu:127-132, 361-436, 842-915): the
// same shape rules for B and T, the same std::invalid_argument messages, the
// same top_k / top_p clamping (done in the C ABI).  Outputs are int32 [B].
//
// Differences a caller can see: the per-row random state is 32 bytes
// (VKWR_SAMPLING_STATE_BYTES), not sizeof(curandStatePhilox4_32_10_t); the
// probability buffer the reference allocates on every call is needed only for
// vocabularies above 65536 (below that the row stays in registers); inputs must
// be contiguous CUDA tensors on the current device.
#include <stdexcept>
#include <string>

#include "vk_torch.h"

using namespace vkt;

namespace {

void check_logits(const at::Tensor& logits) {
  if (logits.dtype() != at::kFloat) {
    throw std::invalid_argument("Logits tensor must be of type float32 (FP32), got " +
                                std::string(logits.dtype().name()) + " !\n");
  }
  check_f32_cuda_contig(logits, "logits");
  check_device(logits, "logits");
}

void check_shape(int64_t B, int64_t T, int64_t V, double temperature) {
  if (!(V > 0 && V <= 1048576 && V % 4 == 0)) {
    throw std::invalid_argument("Vocabulary size must be multiple of 4, and no larger than 1048576, got " +
                                std::to_string(V) + " !\n");
  }
  if (!(B > 0 && T > 0)) {
    throw std::invalid_argument("B and T must be positive, got B=" + std::to_string(B) +
                                ", T=" + std::to_string(T) + " !\n");
  }
  if (!(temperature >= 0.001 && temperature <= 1000)) {
    throw std::invalid_argument("Temperature outside range, got " + std::to_string(temperature) +
                                ", expect [0.001, 1000]!\n");
  }
}

void check_states(const at::Tensor& states, int64_t B) {
  TORCH_CHECK(states.is_cuda() && states.is_contiguous(), "states must be a contiguous CUDA tensor");
  check_device(states, "states");
  TORCH_CHECK(states.nbytes() >= (size_t)B * VKWR_SAMPLING_STATE_BYTES, "states holds ", states.nbytes(),
              " bytes, need ", B * VKWR_SAMPLING_STATE_BYTES, " for B=", B, " (setup_rand(seed, B))");
}

// Probability buffer for vocabularies the kernel cannot keep in registers.
at::Tensor scratch_for(const at::Tensor& logits, int64_t B, int64_t V) {
  if (V <= 65536) return at::Tensor();
  return at::empty({B, V}, logits.options());
}

float* opt_ptr(const at::Tensor& t) { return t.defined() ? ptr<float>(t) : nullptr; }

at::Tensor setup_rand(int64_t seed, int64_t B) {
  TORCH_CHECK(B > 0 && B <= 0x7fffffff, "B must be positive, got ", B);
  auto state = at::zeros({B * VKWR_SAMPLING_STATE_BYTES},
                         at::TensorOptions().dtype(at::kChar).device(at::kCUDA, c10::hip::current_device()));
  check_status(vkwr_sampling_setup_rand(seed, (int)B, state.data_ptr(), stream()), "setup_rand");
  return state;
}

at::Tensor temperature_topk_topp(at::Tensor& logits, at::Tensor& states, at::Scalar temperature, int64_t top_k,
                                 at::Scalar top_p) {
  check_logits(logits);
  const int64_t V = logits.size(-1);
  const int64_t B = logits.dim() >= 2 ? logits.size(0) : 1;
  const int64_t T = logits.dim() == 3 ? logits.size(1) : 1;
  const double temp = temperature.toDouble();
  check_shape(B, T, V, temp);
  check_states(states, B);
  check_fits_int(B * T, "B*T");
  auto out = at::empty({B}, logits.options().dtype(at::kInt));
  auto scratch = scratch_for(logits, B, V);
  const int k = (int)std::max<int64_t>(std::min<int64_t>(top_k, 0x7fffffff), -1);
  check_status(vkwr_sampling_temperature_topk_topp((int)B, (int)T, (int)V, ptr<float>(logits), states.data_ptr(),
                                                   ptr<int32_t>(out), opt_ptr(scratch), temp, k,
                                                   top_p.toDouble(), stream()),
               "temperature_topk_topp");
  return out;
}

at::Tensor repetition_topk_topp(at::Tensor& logits, at::Tensor& penalties, at::Tensor& states,
                                at::Scalar presence_penalty, at::Scalar repetition_penalty,
                                at::Scalar penalty_decay, at::Scalar temperature, int64_t top_k, at::Scalar top_p) {
  check_logits(logits);
  const int64_t V = logits.size(-1);
  const int64_t B = penalties.dim() == 2 ? penalties.size(0) : 1;
  const int64_t T = logits.dim() == 3 ? logits.size(1) : 1;
  const double temp = temperature.toDouble();
  check_shape(B, T, V, temp);
  check_f32_cuda_contig(penalties, "penalties");
  check_device(penalties, "penalties");
  TORCH_CHECK(penalties.numel() == B * V, "penalties must hold B*V = ", B * V, " values, got ", penalties.numel());
  TORCH_CHECK(logits.numel() == B * T * V, "logits must hold B*T*V = ", B * T * V, " values, got ",
              logits.numel());
  check_states(states, B);
  check_fits_int(B * T, "B*T");
  auto out = at::empty({B}, logits.options().dtype(at::kInt));
  auto scratch = scratch_for(logits, B, V);
  const int k = (int)std::max<int64_t>(std::min<int64_t>(top_k, 0x7fffffff), -1);
  check_status(vkwr_sampling_repetition_topk_topp((int)B, (int)T, (int)V, ptr<float>(logits), ptr<float>(penalties),
                                                  states.data_ptr(), ptr<int32_t>(out), opt_ptr(scratch),
                                                  presence_penalty.toDouble(), repetition_penalty.toDouble(),
                                                  penalty_decay.toDouble(), temp, k, top_p.toDouble(), stream()),
               "repetition_topk_topp");
  return out;
}

}  // namespace

TORCH_LIBRARY(vkwr_sampling, m) {
  m.def("setup_rand(int seed, int B) -> Tensor");
  m.impl("setup_rand", &setup_rand);
  m.def(
      "temperature_topk_topp(Tensor logits, Tensor states, "
      "Scalar temperature, int top_k, Scalar top_p) -> Tensor");
  m.impl("temperature_topk_topp", c10::kCUDA, &temperature_topk_topp);
  m.def(
      "repetition_topk_topp(Tensor logits, Tensor penalties, Tensor states, "
      "Scalar presence_penalty, Scalar repetition_penalty, Scalar penalty_decay, "
      "Scalar temperature, int top_k, Scalar top_p) -> Tensor");
  m.impl("repetition_topk_topp", c10::kCUDA, &repetition_topk_topp);
}

VKT_PYMODULE(_sampling_C)
