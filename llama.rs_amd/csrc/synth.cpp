// Synthetic Qwen2 models: random-init weights from a seed, quantized with the
// reference's load-time recipes (maybe_quantize, src/loader.rs:406-447).
//
// Every tensor row has its own SplitMix64 stream keyed by (seed, tensor index,
// row), so generation is deterministic for any thread count.  Normals come
// from Box-Muller in f32 with glibc logf/sqrtf/cosf/sinf.  Matrices and
// biases are N(0, std); RMSNorm gains are 1 + N(0, std) so the residual
// stream keeps its scale through the layers (gains drawn around zero would
// collapse it and make greedy ties likely).
#include "synth.h"

#include <cmath>
#include <cstring>
#include <thread>

#include "quantize.h"

namespace llrs {

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct SplitMix64 {
  uint64_t s;
  uint64_t next() {
    s += 0x9E3779B97F4A7C15ull;
    return mix64(s);
  }
};

// N(0,1) samples into out[0..n) from the stream of (seed, tensor, row).
void synth_normals(uint64_t seed, uint64_t tensor, uint64_t row, float *out, size_t n) {
  SplitMix64 g{mix64(seed + 0x9E3779B97F4A7C15ull * (tensor + 1)) ^
               mix64((row + 1) * 0xD1B54A32D192ED03ull)};
  const float two_pi = 6.28318530717958647692f;
  for (size_t i = 0; i < n; i += 2) {
    float u1 = (float)((g.next() >> 40) + 1) * 5.9604644775390625e-8f;  // (0, 1]
    float u2 = (float)(g.next() >> 40) * 5.9604644775390625e-8f;        // [0, 1)
    float r = sqrtf(-2.0f * logf(u1));
    float th = two_pi * u2;
    out[i] = r * cosf(th);
    if (i + 1 < n) out[i + 1] = r * sinf(th);
  }
}

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

// The tensor type maybe_quantize produces for `name` (src/loader.rs:406-447),
// after the quantizers' own fallbacks (src/quant.rs:190-259).
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
      want = LLRS_Q6_K;
  }
  if (want == LLRS_Q4_K && cols % 256) want = LLRS_Q5_0;
  if (want == LLRS_Q6_K && cols % 256) want = LLRS_Q8_0;
  if ((want == LLRS_Q5_0 || want == LLRS_Q8_0) && cols % 32) want = LLRS_F32;
  return want;
}

int synth_tensor(const llrs_synth_config &c, size_t index, const SynthSpec &spec,
                 GgufOutTensor &out) {
  out.name = spec.name;
  const float sd = c.weight_std;
  if (spec.kind != SynthSpec::MATRIX) {
    out.dims = {spec.cols};
    out.type = LLRS_F32;
    std::vector<float> v(spec.cols);
    synth_normals(c.seed, index, 0, v.data(), v.size());
    for (auto &x : v) x = spec.kind == SynthSpec::GAIN ? 1.0f + sd * x : sd * x;
    out.bytes.resize(v.size() * 4);
    memcpy(out.bytes.data(), v.data(), out.bytes.size());
    return LLRS_OK;
  }
  uint32_t ty = recipe_type(c.recipe, spec.name, spec.cols);
  out.dims = {spec.cols, spec.rows};
  out.type = ty;
  size_t rb = ty == LLRS_F32 ? spec.cols * 4 : row_bytes(ty, spec.cols);
  try {
    out.bytes.assign(rb * spec.rows, 0);
  } catch (...) {
    return set_error(LLRS_E_OOM, "out of host memory for %s", spec.name.c_str());
  }
  unsigned nt = c.threads > 0 ? (unsigned)c.threads : std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  if (nt > spec.rows) nt = (unsigned)spec.rows ? (unsigned)spec.rows : 1;
  auto work = [&](size_t r0, size_t r1) {
    std::vector<float> vals(spec.cols);
    std::vector<uint8_t> q;
    for (size_t r = r0; r < r1; r++) {
      synth_normals(c.seed, index, r, vals.data(), spec.cols);
      for (auto &x : vals) x *= sd;
      if (ty == LLRS_F32) {
        memcpy(out.bytes.data() + r * rb, vals.data(), rb);
      } else {
        quantize_rows(ty, vals.data(), 1, spec.cols, q);  // ty is final: no further fallback
        memcpy(out.bytes.data() + r * rb, q.data(), rb);
      }
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
