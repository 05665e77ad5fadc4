// Synthetic Qwen2 models: random-init weights from a seed, quantized with the
// reference's load-time recipes (maybe_quantize, src/loader.rs:406-447).
//
// Element e (row-major) of the tensor with index t is
//   std * z(seed, t, e)        (matrices, biases)
//   1 + std * z(seed, t, e)    (RMSNorm gains, so the residual stream keeps its
//                               scale; gains drawn around zero would collapse it)
// where z is a Box-Muller normal from a counter-based hash (quant_encode.h).
// The host path here and the GPU path (launch_synth_encode) use the same
// functions, so a GGUF written here holds exactly the bytes that
// llrs_model_synthetic builds in HBM.
#include "synth.h"

#include <cstring>
#include <thread>

#include "quant_encode.h"
#include "quantize.h"

namespace llrs {

std::vector<SynthSpec> synth_specs(const llrs_synth_config &c) {
  std::vector<SynthSpec> v;
  uint64_t H = c.hidden_size, F = c.intermediate_size, V = c.vocab_size;
  uint64_t hd = c.num_attention_heads ? H / c.num_attention_heads : 0;
  uint64_t KV = c.num_key_value_heads * hd;
  auto mat = [&](std::string n, uint64_t rows, uint64_t cols) {
    v.push_back({n, rows, cols, SynthSpec::MATRIX});
  };
  auto vec = [&](std::string n, uint64_t len, SynthSpec::Kind k) { v.push_back({n, 1, len, k}); };
  mat("token_embd.weight", V, H);
  for (size_t i = 0; i < c.num_hidden_layers; i++) {
    std::string p = "blk." + std::to_string(i) + ".";
    vec(p + "attn_norm.weight", H, SynthSpec::GAIN);
    mat(p + "attn_q.weight", H, H);
    vec(p + "attn_q.bias", H, SynthSpec::BIAS);
    mat(p + "attn_k.weight", KV, H);
    vec(p + "attn_k.bias", KV, SynthSpec::BIAS);
    mat(p + "attn_v.weight", KV, H);
    vec(p + "attn_v.bias", KV, SynthSpec::BIAS);
    mat(p + "attn_output.weight", H, H);
    vec(p + "ffn_norm.weight", H, SynthSpec::GAIN);
    mat(p + "ffn_gate.weight", F, H);
    mat(p + "ffn_up.weight", F, H);
    mat(p + "ffn_down.weight", H, F);
  }
  vec("output_norm.weight", H, SynthSpec::GAIN);
  if (!c.tie_word_embeddings) mat("output.weight", V, H);
  return v;
}

uint32_t recipe_type(int recipe, const std::string &name, uint64_t cols) {
  if (recipe == LLRS_QUANT_NONE) return LLRS_F32;
  uint32_t want = LLRS_Q4_K;
  if (recipe == LLRS_QUANT_Q4KM) {
    if (name.find("embed_tokens") != std::string::npos || name == "token_embd.weight" ||
        name == "lm_head.weight" || name == "output.weight" ||
        name.find("attn.v_proj.weight") != std::string::npos ||
        name.find("attn_v.weight") != std::string::npos)
      want = LLRS_Q8_0;
    else if (name.find("mlp.down_proj.weight") != std::string::npos ||
             name.find("ffn_down.weight") != std::string::npos)
      // Down projections stay at Q6_K in the reference's recipe.
      want = LLRS_Q6_K;
  }
  return final_quant_type(want, cols);
}

uint32_t synth_type(const llrs_synth_config &c, const SynthSpec &spec) {
  return spec.kind == SynthSpec::MATRIX ? recipe_type(c.recipe, spec.name, spec.cols) : LLRS_F32;
}

int synth_tensor(const llrs_synth_config &c, size_t index, const SynthSpec &spec,
                 GgufOutTensor &out) {
  out.name = spec.name;
  uint32_t ty = synth_type(c, spec);
  out.type = ty;
  out.dims = spec.kind == SynthSpec::MATRIX ? std::vector<uint64_t>{spec.cols, spec.rows}
                                            : std::vector<uint64_t>{spec.cols};
  size_t rb = ty == LLRS_F32 ? spec.cols * 4 : row_bytes(ty, spec.cols);
  try {
    out.bytes.assign(rb * spec.rows, 0);
  } catch (...) {
    return set_error(LLRS_E_OOM, "out of host memory for %s", spec.name.c_str());
  }
  uint64_t key = enc::tensor_key(c.seed, index);
  bool gain = spec.kind == SynthSpec::GAIN;
  unsigned nt = c.threads > 0 ? (unsigned)c.threads : std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  if (nt > spec.rows) nt = (unsigned)spec.rows;
  auto work = [&](size_t r0, size_t r1) {
    std::vector<float> vals(spec.cols);
    for (size_t r = r0; r < r1; r++) {
      for (size_t j = 0; j < spec.cols; j++)
        vals[j] = enc::synth_value(key, r * spec.cols + j, c.weight_std, gain);
      encode_row(ty, vals.data(), spec.cols, out.bytes.data() + r * rb);
    }
  };
  std::vector<std::thread> th;
  size_t per = (spec.rows + nt - 1) / nt;
  for (unsigned t = 0; t < nt; t++) {
    size_t r0 = t * per, r1 = std::min<size_t>(spec.rows, r0 + per);
    if (r0 >= r1) break;
    th.emplace_back(work, r0, r1);
  }
  for (auto &t : th) t.join();
  return LLRS_OK;
}

}  // namespace llrs
