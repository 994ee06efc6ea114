// pybind11 module `qwen_megakernel_C`: the reference's extension boundary
// (Tools/megakernel/qwen_ops.cpp:30-171) over the MI355X engine's C-ABI.
//
// decode / generate_nosync / abi_version keep the reference's names, argument
// order (24 / 25 positional arguments, Model/Qwen06B_architecture.py:304-376)
// and return values (a device int32 tensor). Each call hands raw device
// pointers and torch's current HIP stream to libqwen_megakernel.so. Unlike the
// reference, every tensor's device, dtype, contiguity and size is checked and a
// violation raises RuntimeError; the pointer-table alignment check of
// qwen_ops.cpp:64-65 is kept.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <string>
#include <tuple>
#include <vector>

#include "qwen_megakernel.h"

namespace {

constexpr int64_t H = 1024, V = 151936, NKV = 8, HD = 128;

void check_dev(const torch::Tensor& t, const char* name, c10::ScalarType dt, int64_t numel = -1) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.scalar_type() == dt, name, " has dtype ", t.scalar_type(), ", expected ", c10::toString(dt));
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  if (numel >= 0) TORCH_CHECK(t.numel() >= numel, name, " has ", t.numel(), " elements, needs ", numel);
}

hipStream_t stream_of(const torch::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void check_rc(int rc, const char* what) {
  if (rc == QWEN_OK) return;
  const char* why = rc == QWEN_ERR_ARG         ? "invalid argument"
                    : rc == QWEN_ERR_DEVICE    ? "unsupported device (needs a 256-CU gfx950 MI355X with cooperative "
                                                 "launch and workgroup w on XCD w % 8)"
                    : rc == QWEN_ERR_LAUNCH    ? "HIP launch or allocation failure"
                    : rc == QWEN_ERR_BAD_TOKEN ? "a forced token id out of range reached the device"
                                               : "device-side timeout";
  TORCH_CHECK(false, "qwen_megakernel_C.", what, " failed: ", why, " (code ", rc, ")");
}

// checks shared by decode / generate_nosync; returns the pointer table
const LDGLayerWeight* check_common(const torch::Tensor& embed_weight, const torch::Tensor& layer_weights_packed,
                                   const torch::Tensor& final_norm_weight, const torch::Tensor& lm_head_weight,
                                   const torch::Tensor& cos_table, const torch::Tensor& sin_table,
                                   const torch::Tensor& k_cache, const torch::Tensor& v_cache,
                                   const torch::Tensor& hidden, const torch::Tensor& norm_out, int num_layers,
                                   int max_seq_len) {
  check_dev(embed_weight, "embed_weight", torch::kHalf, V * H);
  TORCH_CHECK(layer_weights_packed.is_cuda() && layer_weights_packed.scalar_type() == torch::kLong,
              "layer_weights_packed must be an int64 GPU tensor");
  TORCH_CHECK(layer_weights_packed.numel() >= (int64_t)num_layers * 12, "layer_weights_packed holds ",
              layer_weights_packed.numel(), " pointers, needs ", num_layers * 12);
  const uintptr_t ptr_val = reinterpret_cast<uintptr_t>(layer_weights_packed.data_ptr());
  TORCH_CHECK(ptr_val % 16 == 0, "layer_weights_packed must be 16-byte aligned (address ends in ", ptr_val % 16, ")");
  check_dev(final_norm_weight, "final_norm_weight", torch::kHalf, H);
  check_dev(lm_head_weight, "lm_head_weight", torch::kHalf, V * H);
  check_dev(cos_table, "cos_table", torch::kHalf, (int64_t)max_seq_len * HD);
  check_dev(sin_table, "sin_table", torch::kHalf, (int64_t)max_seq_len * HD);
  check_dev(k_cache, "k_cache", torch::kHalf, (int64_t)num_layers * NKV * max_seq_len * HD);
  check_dev(v_cache, "v_cache", torch::kHalf, (int64_t)num_layers * NKV * max_seq_len * HD);
  check_dev(hidden, "hidden", torch::kHalf, H);
  check_dev(norm_out, "norm_out", torch::kFloat, H);
  return reinterpret_cast<const LDGLayerWeight*>(layer_weights_packed.data_ptr());
}

int abi_version() { return qwen_abi_version(); }

std::string built_torch_version() { return TORCH_VERSION; }

torch::Tensor decode(int input_token_id, torch::Tensor embed_weight, torch::Tensor layer_weights_packed,
                     torch::Tensor final_norm_weight, torch::Tensor lm_head_weight, torch::Tensor cos_table,
                     torch::Tensor sin_table, torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor hidden,
                     torch::Tensor act, torch::Tensor res, torch::Tensor q, torch::Tensor k, torch::Tensor v,
                     torch::Tensor attn_out, torch::Tensor mlp_inter, torch::Tensor norm_out, torch::Tensor bmax_vals,
                     torch::Tensor bmax_idxs, int num_layers, int position, int max_seq_len, float attn_scale) {
  const LDGLayerWeight* tab = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight,
                                           cos_table, sin_table, k_cache, v_cache, hidden, norm_out, num_layers,
                                           max_seq_len);
  TORCH_CHECK(input_token_id >= 0 && input_token_id < V, "input_token_id ", input_token_id, " out of range");
  TORCH_CHECK(position >= 0 && position < max_seq_len, "position ", position, " outside [0, ", max_seq_len, ")");
  auto out = torch::zeros({1}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  const int rc = launch_ldg_decode_direct(
      input_token_id, out.data_ptr<int>(), embed_weight.data_ptr(), tab, final_norm_weight.data_ptr(),
      lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
      hidden.data_ptr(), act.data_ptr(), res.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), attn_out.data_ptr(),
      mlp_inter.data_ptr(), norm_out.data_ptr(), bmax_vals.data_ptr(), bmax_idxs.data_ptr(), num_layers, position,
      max_seq_len, attn_scale, stream_of(embed_weight));
  check_rc(rc, "decode");
  return out;
}

torch::Tensor generate_nosync(int first_token_id, int num_steps, torch::Tensor embed_weight,
                              torch::Tensor layer_weights_packed, torch::Tensor final_norm_weight,
                              torch::Tensor lm_head_weight, torch::Tensor cos_table, torch::Tensor sin_table,
                              torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor hidden, torch::Tensor act,
                              torch::Tensor res, torch::Tensor q, torch::Tensor k, torch::Tensor v,
                              torch::Tensor attn_out, torch::Tensor mlp_inter, torch::Tensor norm_out,
                              torch::Tensor bmax_vals, torch::Tensor bmax_idxs, int num_layers, int start_position,
                              int max_seq_len, float attn_scale) {
  const LDGLayerWeight* tab = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight,
                                           cos_table, sin_table, k_cache, v_cache, hidden, norm_out, num_layers,
                                           max_seq_len);
  TORCH_CHECK(first_token_id >= 0 && first_token_id < V, "first_token_id ", first_token_id, " out of range");
  TORCH_CHECK(num_steps >= 1, "num_steps must be >= 1");
  TORCH_CHECK(start_position >= 0 && (int64_t)start_position + num_steps <= max_seq_len, "positions [",
              start_position, ", ", (int64_t)start_position + num_steps, ") exceed max_seq_len ", max_seq_len);
  auto out = torch::zeros({num_steps}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  const int rc = launch_ldg_generate_nosync(
      first_token_id, num_steps, embed_weight.data_ptr(), tab, final_norm_weight.data_ptr(), lm_head_weight.data_ptr(),
      cos_table.data_ptr(), sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), hidden.data_ptr(),
      act.data_ptr(), res.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), attn_out.data_ptr(),
      mlp_inter.data_ptr(), norm_out.data_ptr(), bmax_vals.data_ptr(), bmax_idxs.data_ptr(), out.data_ptr<int>(),
      num_layers, start_position, max_seq_len, attn_scale, stream_of(embed_weight));
  check_rc(rc, "generate_nosync");
  return out;
}

// generate_nosync with teacher forcing and per-step logits / hidden outputs
torch::Tensor generate_ex(int first_token_id, int num_steps, c10::optional<torch::Tensor> forced_tokens,
                          torch::Tensor embed_weight, torch::Tensor layer_weights_packed,
                          torch::Tensor final_norm_weight, torch::Tensor lm_head_weight, torch::Tensor cos_table,
                          torch::Tensor sin_table, torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor hidden,
                          torch::Tensor norm_out, c10::optional<torch::Tensor> logits_out,
                          c10::optional<torch::Tensor> hidden_steps, int num_layers, int start_position,
                          int max_seq_len, float attn_scale) {
  const LDGLayerWeight* tab = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight,
                                           cos_table, sin_table, k_cache, v_cache, hidden, norm_out, num_layers,
                                           max_seq_len);
  TORCH_CHECK(first_token_id >= 0 && first_token_id < V, "first_token_id ", first_token_id, " out of range");
  TORCH_CHECK(num_steps >= 1, "num_steps must be >= 1");
  TORCH_CHECK(start_position >= 0 && (int64_t)start_position + num_steps <= max_seq_len, "positions exceed max_seq_len");
  const int* forced = nullptr;
  if (forced_tokens.has_value()) {
    check_dev(*forced_tokens, "forced_tokens", torch::kInt32, num_steps);
    auto host = forced_tokens->cpu();
    auto acc = host.accessor<int, 1>();
    for (int i = 1; i < num_steps; ++i)
      TORCH_CHECK(acc[i] >= 0 && acc[i] < V, "forced_tokens[", i, "] = ", acc[i], " out of range");
    forced = forced_tokens->data_ptr<int>();
  }
  float* lo = nullptr;
  float* hs = nullptr;
  if (logits_out.has_value()) {
    check_dev(*logits_out, "logits_out", torch::kFloat, (int64_t)num_steps * V);
    lo = logits_out->data_ptr<float>();
  }
  if (hidden_steps.has_value()) {
    check_dev(*hidden_steps, "hidden_steps", torch::kFloat, (int64_t)num_steps * H);
    hs = hidden_steps->data_ptr<float>();
  }
  auto out = torch::zeros({num_steps}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  const int rc = qwen_generate_ex(first_token_id, num_steps, forced, embed_weight.data_ptr(), tab,
                                  final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(),
                                  sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), hidden.data_ptr(),
                                  norm_out.data_ptr(), out.data_ptr<int>(), lo, hs, num_layers, start_position,
                                  max_seq_len, attn_scale, stream_of(embed_weight));
  check_rc(rc, "generate_ex");
  return out;
}

// generate_nosync that ends at eos_token_id; returns (ids int32[num_steps], count int32[1]),
// both on the device: ids[0 .. count) were generated, the rest are -1
std::tuple<torch::Tensor, torch::Tensor> generate_until(int first_token_id, int num_steps, int eos_token_id,
                                                        torch::Tensor embed_weight, torch::Tensor layer_weights_packed,
                                                        torch::Tensor final_norm_weight, torch::Tensor lm_head_weight,
                                                        torch::Tensor cos_table, torch::Tensor sin_table,
                                                        torch::Tensor k_cache, torch::Tensor v_cache,
                                                        torch::Tensor hidden, torch::Tensor norm_out, int num_layers,
                                                        int start_position, int max_seq_len, float attn_scale) {
  const LDGLayerWeight* tab = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight,
                                           cos_table, sin_table, k_cache, v_cache, hidden, norm_out, num_layers,
                                           max_seq_len);
  TORCH_CHECK(first_token_id >= 0 && first_token_id < V, "first_token_id ", first_token_id, " out of range");
  TORCH_CHECK(eos_token_id >= 0 && eos_token_id < V, "eos_token_id ", eos_token_id, " out of range");
  TORCH_CHECK(num_steps >= 1, "num_steps must be >= 1");
  TORCH_CHECK(start_position >= 0 && (int64_t)start_position + num_steps <= max_seq_len, "positions exceed max_seq_len");
  auto out = torch::full({num_steps}, -1, torch::dtype(torch::kInt32).device(embed_weight.device()));
  auto count = torch::zeros({1}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  const int rc = qwen_generate_until(first_token_id, num_steps, eos_token_id, embed_weight.data_ptr(), tab,
                                     final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(),
                                     sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), hidden.data_ptr(),
                                     norm_out.data_ptr(), out.data_ptr<int>(), count.data_ptr<int>(), num_layers,
                                     start_position, max_seq_len, attn_scale, stream_of(embed_weight));
  check_rc(rc, "generate_until");
  return {out, count};
}

// one token sampled from fp32 logits (device int32[1])
torch::Tensor sample(torch::Tensor logits, double temperature, int64_t top_k, double top_p, uint64_t seed,
                     int64_t step) {
  check_dev(logits, "logits", torch::kFloat);
  TORCH_CHECK(logits.numel() >= 1 && logits.numel() <= INT32_MAX, "logits must hold 1 .. 2^31-1 values");
  TORCH_CHECK(top_k >= 0 && top_k <= INT32_MAX, "top_k must be >= 0");
  TORCH_CHECK(step >= 0 && step <= UINT32_MAX, "step must fit 32 bits");
  auto out = torch::empty({1}, torch::dtype(torch::kInt32).device(logits.device()));
  check_rc(qwen_sample(logits.data_ptr<float>(), (int)logits.numel(), (float)temperature, (int)top_k, (float)top_p,
                       seed, (unsigned)step, out.data_ptr<int>(), stream_of(logits)),
           "sample");
  return out;
}

// generate_until with sampling; returns (ids int32[num_steps], count int32[1]) on the device
std::tuple<torch::Tensor, torch::Tensor> generate_sampled(
    int first_token_id, int num_steps, int eos_token_id, torch::Tensor embed_weight,
    torch::Tensor layer_weights_packed, torch::Tensor final_norm_weight, torch::Tensor lm_head_weight,
    torch::Tensor cos_table, torch::Tensor sin_table, torch::Tensor k_cache, torch::Tensor v_cache,
    torch::Tensor hidden, torch::Tensor norm_out, int num_layers, int start_position, int max_seq_len,
    float attn_scale, double temperature, int64_t top_k, double top_p, uint64_t seed) {
  const LDGLayerWeight* tab = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight,
                                           cos_table, sin_table, k_cache, v_cache, hidden, norm_out, num_layers,
                                           max_seq_len);
  TORCH_CHECK(first_token_id >= 0 && first_token_id < V, "first_token_id ", first_token_id, " out of range");
  TORCH_CHECK(eos_token_id >= -1 && eos_token_id < V, "eos_token_id ", eos_token_id, " out of range");
  TORCH_CHECK(num_steps >= 1, "num_steps must be >= 1");
  TORCH_CHECK(start_position >= 0 && (int64_t)start_position + num_steps <= max_seq_len, "positions exceed max_seq_len");
  TORCH_CHECK(top_k >= 0 && top_k <= INT32_MAX, "top_k must be >= 0");
  auto out = torch::full({num_steps}, -1, torch::dtype(torch::kInt32).device(embed_weight.device()));
  auto count = torch::zeros({1}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  const int rc = qwen_generate_sampled(
      first_token_id, num_steps, eos_token_id, embed_weight.data_ptr(), tab, final_norm_weight.data_ptr(),
      lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
      hidden.data_ptr(), norm_out.data_ptr(), out.data_ptr<int>(), count.data_ptr<int>(), num_layers, start_position,
      max_seq_len, attn_scale, (float)temperature, (int)top_k, (float)top_p, seed, stream_of(embed_weight));
  check_rc(rc, "generate_sampled");
  return {out, count};
}

// batched prefill of `ids` (int32 device tensor) at start_position ..; writes K/V and hidden
void prefill(torch::Tensor ids, torch::Tensor embed_weight, torch::Tensor layer_weights_packed,
             torch::Tensor cos_table, torch::Tensor sin_table, torch::Tensor k_cache, torch::Tensor v_cache,
             torch::Tensor hidden, int num_layers, int start_position, int max_seq_len, float attn_scale) {
  check_dev(ids, "ids", torch::kInt32);
  const int64_t n = ids.numel();
  TORCH_CHECK(n >= 1, "prefill needs at least one id");
  TORCH_CHECK(start_position >= 0 && start_position + n <= max_seq_len, "positions [", start_position, ", ",
              start_position + n, ") exceed max_seq_len ", max_seq_len);
  check_dev(embed_weight, "embed_weight", torch::kHalf, V * H);
  TORCH_CHECK(layer_weights_packed.is_cuda() && layer_weights_packed.scalar_type() == torch::kLong,
              "layer_weights_packed must be an int64 GPU tensor");
  TORCH_CHECK(layer_weights_packed.numel() >= (int64_t)num_layers * 12, "layer_weights_packed too small");
  TORCH_CHECK(reinterpret_cast<uintptr_t>(layer_weights_packed.data_ptr()) % 16 == 0,
              "layer_weights_packed must be 16-byte aligned");
  check_dev(cos_table, "cos_table", torch::kHalf, (int64_t)max_seq_len * HD);
  check_dev(sin_table, "sin_table", torch::kHalf, (int64_t)max_seq_len * HD);
  check_dev(k_cache, "k_cache", torch::kHalf, (int64_t)num_layers * NKV * max_seq_len * HD);
  check_dev(v_cache, "v_cache", torch::kHalf, (int64_t)num_layers * NKV * max_seq_len * HD);
  check_dev(hidden, "hidden", torch::kHalf, H);
  check_rc(qwen_prefill(ids.data_ptr<int>(), (int)n, embed_weight.data_ptr(),
                        reinterpret_cast<const LDGLayerWeight*>(layer_weights_packed.data_ptr()),
                        cos_table.data_ptr(), sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                        hidden.data_ptr(), num_layers, start_position, max_seq_len, attn_scale, stream_of(ids)),
           "prefill");
}

// wall-clock ticks at the start and every grid barrier of the last prefill (profiling aid)
std::vector<int64_t> prefill_timestamps() {
  std::vector<unsigned long long> buf(2 + 5 * 28);
  check_rc(qwen_prefill_timestamps(buf.data(), (int)buf.size()), "prefill_timestamps");
  return std::vector<int64_t>(buf.begin(), buf.end());
}

torch::Tensor lm_head_argmax(torch::Tensor hidden, torch::Tensor weight, c10::optional<torch::Tensor> logits_out) {
  check_dev(hidden, "hidden", torch::kHalf, H);
  check_dev(weight, "weight", torch::kHalf, V * H);
  float* lo = nullptr;
  if (logits_out.has_value()) {
    check_dev(*logits_out, "logits_out", torch::kFloat, V);
    lo = logits_out->data_ptr<float>();
  }
  auto out = torch::zeros({1}, torch::dtype(torch::kInt32).device(weight.device()));
  check_rc(qwen_lm_head_argmax(hidden.data_ptr(), weight.data_ptr(), out.data_ptr<int>(), lo, stream_of(weight)),
           "lm_head_argmax");
  return out;
}

torch::Tensor lm_head_sample(torch::Tensor hidden, torch::Tensor weight, double temperature, int64_t top_k,
                             double top_p, uint64_t seed, int64_t position, c10::optional<torch::Tensor> logits_out) {
  check_dev(hidden, "hidden", torch::kHalf, H);
  check_dev(weight, "weight", torch::kHalf, V * H);
  float* lo = nullptr;
  if (logits_out.has_value()) {
    check_dev(*logits_out, "logits_out", torch::kFloat, V);
    lo = logits_out->data_ptr<float>();
  }
  TORCH_CHECK(temperature > 0 && top_k >= 0 && position >= 0 && position < (1LL << 31),
              "lm_head_sample: temperature > 0, top_k >= 0, position >= 0");
  auto out = torch::zeros({1}, torch::dtype(torch::kInt32).device(weight.device()));
  check_rc(qwen_lm_head_sample(hidden.data_ptr(), weight.data_ptr(), (float)temperature, (int)top_k, (float)top_p, seed,
                               (int)position, out.data_ptr<int>(), lo, stream_of(weight)),
           "lm_head_sample");
  return out;
}

torch::Tensor mlp_block(torch::Tensor x, torch::Tensor post_norm, torch::Tensor gate, torch::Tensor up,
                        torch::Tensor down) {
  check_dev(x, "x", torch::kHalf, H);
  check_dev(post_norm, "post_norm", torch::kHalf, H);
  check_dev(gate, "gate", torch::kHalf, 3072 * H);
  check_dev(up, "up", torch::kHalf, 3072 * H);
  check_dev(down, "down", torch::kHalf, 3072 * H);
  auto y = torch::empty({H}, torch::dtype(torch::kFloat).device(x.device()));
  check_rc(qwen_mlp_block(x.data_ptr(), post_norm.data_ptr(), gate.data_ptr(), up.data_ptr(), down.data_ptr(),
                          y.data_ptr<float>(), stream_of(x)),
           "mlp_block");
  return y;
}

int last_error() { return qwen_last_error(); }

void set_trace(c10::optional<torch::Tensor> buf, int token) {
  if (!buf.has_value()) {
    check_rc(qwen_set_trace(nullptr, 0, -1), "set_trace");
    return;
  }
  TORCH_CHECK(buf->is_cuda() && buf->scalar_type() == torch::kLong && buf->is_contiguous(),
              "trace buffer must be a contiguous int64 GPU tensor");
  TORCH_CHECK(buf->numel() > 0, "trace buffer is empty");
  check_rc(qwen_set_trace(reinterpret_cast<unsigned long long*>(buf->data_ptr<int64_t>()), buf->numel(), token),
           "set_trace");
}

void set_wait_deadline_us(int64_t us) { check_rc(qwen_set_wait_deadline_us(us), "set_wait_deadline_us"); }

}  // namespace

PYBIND11_MODULE(qwen_megakernel_C, m) {
  m.def("decode", &decode, "Qwen3 single token decode");
  m.def("generate_nosync", &generate_nosync, "Qwen3 on-device greedy generation (one launch, no host sync)");
  m.def("abi_version", &abi_version, "ABI version of the extension (2)");
  m.def("built_torch_version", &built_torch_version, "torch version the extension was built against");
  m.def("generate_ex", &generate_ex, "generate with forced tokens and per-step logits / hidden outputs",
        pybind11::arg("first_token_id"), pybind11::arg("num_steps"), pybind11::arg("forced_tokens"),
        pybind11::arg("embed_weight"), pybind11::arg("layer_weights_packed"), pybind11::arg("final_norm_weight"),
        pybind11::arg("lm_head_weight"), pybind11::arg("cos_table"), pybind11::arg("sin_table"),
        pybind11::arg("k_cache"), pybind11::arg("v_cache"), pybind11::arg("hidden"), pybind11::arg("norm_out"),
        pybind11::arg("logits_out"), pybind11::arg("hidden_steps"), pybind11::arg("num_layers"),
        pybind11::arg("start_position"), pybind11::arg("max_seq_len"), pybind11::arg("attn_scale"));
  m.def("generate_until", &generate_until, "on-device greedy generation that ends at eos_token_id",
        pybind11::arg("first_token_id"), pybind11::arg("num_steps"), pybind11::arg("eos_token_id"),
        pybind11::arg("embed_weight"), pybind11::arg("layer_weights_packed"), pybind11::arg("final_norm_weight"),
        pybind11::arg("lm_head_weight"), pybind11::arg("cos_table"), pybind11::arg("sin_table"),
        pybind11::arg("k_cache"), pybind11::arg("v_cache"), pybind11::arg("hidden"), pybind11::arg("norm_out"),
        pybind11::arg("num_layers"), pybind11::arg("start_position"), pybind11::arg("max_seq_len"),
        pybind11::arg("attn_scale"));
  m.def("lm_head_argmax", &lm_head_argmax, "isolated lm_head GEMV + argmax", pybind11::arg("hidden"),
        pybind11::arg("weight"), pybind11::arg("logits_out") = pybind11::none());
  m.def("lm_head_sample", &lm_head_sample, "isolated lm_head GEMV + the decode kernel's top-k draw",
        pybind11::arg("hidden"), pybind11::arg("weight"), pybind11::arg("temperature"), pybind11::arg("top_k"),
        pybind11::arg("top_p"), pybind11::arg("seed"), pybind11::arg("position"),
        pybind11::arg("logits_out") = pybind11::none());
  m.def("mlp_block", &mlp_block, "isolated RMSNorm + SwiGLU MLP + residual");
  m.def("prefill_timestamps", &prefill_timestamps, "wall-clock ticks (100 MHz) at the start and at every grid "
        "barrier of the last prefill: start, embedding, then QKV / attention / o_proj / gate-up / down per layer");
  m.def("prefill", &prefill, "batched prefill of a prompt (MFMA): writes K/V of every position and hidden",
        pybind11::arg("ids"), pybind11::arg("embed_weight"), pybind11::arg("layer_weights_packed"),
        pybind11::arg("cos_table"), pybind11::arg("sin_table"), pybind11::arg("k_cache"), pybind11::arg("v_cache"),
        pybind11::arg("hidden"), pybind11::arg("num_layers"), pybind11::arg("start_position"),
        pybind11::arg("max_seq_len"), pybind11::arg("attn_scale"));
  m.def("sample", &sample, "one token from fp32 logits: temperature, top-k, top-p, Philox Gumbel-max draw",
        pybind11::arg("logits"), pybind11::arg("temperature"), pybind11::arg("top_k") = 0,
        pybind11::arg("top_p") = 1.0, pybind11::arg("seed") = 0, pybind11::arg("step") = 0);
  m.def("generate_sampled", &generate_sampled, "on-device sampled generation (no host sync), ends at eos_token_id "
        "(-1: never)",
        pybind11::arg("first_token_id"), pybind11::arg("num_steps"), pybind11::arg("eos_token_id"),
        pybind11::arg("embed_weight"), pybind11::arg("layer_weights_packed"), pybind11::arg("final_norm_weight"),
        pybind11::arg("lm_head_weight"), pybind11::arg("cos_table"), pybind11::arg("sin_table"),
        pybind11::arg("k_cache"), pybind11::arg("v_cache"), pybind11::arg("hidden"), pybind11::arg("norm_out"),
        pybind11::arg("num_layers"), pybind11::arg("start_position"), pybind11::arg("max_seq_len"),
        pybind11::arg("attn_scale"), pybind11::arg("temperature"), pybind11::arg("top_k"), pybind11::arg("top_p"),
        pybind11::arg("seed"));
  m.def("last_error", &last_error, "synchronize and return the device-side error state (0 = ok)");
  m.def("set_trace", &set_trace, "record per-stage device timestamps of one token into an int64 GPU tensor "
        "[256, fins, events] (None to stop)", pybind11::arg("buf"), pybind11::arg("token") = 0);
  m.def("trace_events", &qwen_trace_events, "events recorded per stage by set_trace");
  m.def("set_wait_deadline_us", &set_wait_deadline_us, "test hook: wall-clock budget of every device-side wait "
        "of later launches (0 = default 0.5 s)");
}
