// Test driver for the sanitizer build of the host parsers: runs one parser of
// the product library's host code on each file given, printing "ok" or
// "rejected: <message>".  Built with AddressSanitizer and UndefinedBehavior-
// Sanitizer by tests/test_fuzz_host.py (g++, host code only); any memory error
// or undefined behaviour aborts with the sanitizer's report.
//
//   fuzz_host gguf FILE...         GgufFile::open + tensor lookup and read
//   fuzz_host json FILE...         the JSON reader
//   fuzz_host config FILE...       LlamaConfig::from_json + validate
//   fuzz_host safetensors DIR...   the SafeTensors store + tensor read
//   fuzz_host eos DIR...           find_eos_tokens
//   fuzz_host quantize FILE...     the Q4_K / Q6_K / Q5_0 / Q8_0 encoders on the
//                                  file's bytes read as f32 values
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/llrs.h"
#include "../../llama.rs_amd/csrc/json.h"

static std::string slurp(const char *path) {
  std::ifstream in(path, std::ios::binary);
  std::stringstream ss;
  ss << in.rdbuf();
  return ss.str();
}

static void report(const char *what, int rc) {
  if (rc == 0)
    printf("%s: ok\n", what);
  else
    printf("%s: rejected: %s\n", what, llrs_last_error());
  fflush(stdout);
}

static int gguf(const char *path) {
  uint32_t ver = 0, ty = 0;
  size_t rows = 0, cols = 0, nb = 0;
  int rc = 0;
  for (const char *name : {"t", "token_embd.weight", "blk.0.attn_q.bias"}) {
    rc = llrs_gguf_read_tensor(path, name, &ver, &ty, &rows, &cols, nullptr, 0, &nb);
    if (rc == 0 && nb < (1u << 26)) {
      std::vector<uint8_t> buf(nb ? nb : 1);
      rc = llrs_gguf_read_tensor(path, name, &ver, &ty, &rows, &cols, buf.data(), buf.size(), &nb);
    }
  }
  return rc;
}

static int safetensors(const char *dir) {
  uint32_t ty = 0;
  size_t shape[2] = {0, 0}, ndim = 0, nb = 0;  // rank <= 2 (the reader rejects others)
  int rc = llrs_safetensors_read_tensor(dir, "w", &ty, shape, &ndim, nullptr, 0, &nb);
  if (rc == 0 && nb < (1u << 26)) {
    std::vector<uint8_t> buf(nb ? nb : 1);
    rc = llrs_safetensors_read_tensor(dir, "w", &ty, shape, &ndim, buf.data(), buf.size(), &nb);
  }
  int fmt = 0;
  char resolved[4096];
  (void)llrs_model_format(dir, &fmt, resolved, sizeof resolved);
  return rc;
}

static int quantize(const char *path) {
  const std::string bytes = slurp(path);
  std::vector<float> v(bytes.size() / 4);
  memcpy(v.data(), bytes.data(), v.size() * 4);
  int rc = 0;
  for (uint32_t t : {LLRS_Q4_K, LLRS_Q6_K, LLRS_Q5_0, LLRS_Q8_0}) {
    const size_t cols = t == LLRS_Q4_K || t == LLRS_Q6_K ? 256 : 32;
    const size_t rows = v.size() / cols;
    size_t need = 0;
    uint32_t out_ty = 0;
    rc = llrs_quantize(t, v.data(), rows, cols, nullptr, 0, &need, &out_ty);
    if (rc) return rc;
    std::vector<uint8_t> out(need ? need : 1);
    rc = llrs_quantize(t, v.data(), rows, cols, out.data(), out.size(), &need, &out_ty);
    if (rc) return rc;
  }
  return rc;
}

int main(int argc, char **argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: fuzz_host MODE FILE...\n");
    return 2;
  }
  const std::string mode = argv[1];
  for (int i = 2; i < argc; i++) {
    printf("== %s\n", argv[i]);
    fflush(stdout);
    int rc = 0;
    if (mode == "gguf") {
      rc = gguf(argv[i]);
    } else if (mode == "json") {
      const std::string s = slurp(argv[i]);
      llrs::JsonValue v;
      std::string err;
      rc = llrs::json_parse(s.data(), s.size(), v, err) ? 0 : -1;
      if (rc) printf("%s: rejected: %s\n", argv[i], err.c_str());
      else printf("%s: ok\n", argv[i]);
      continue;
    } else if (mode == "config") {
      llrs_model_config c;
      rc = llrs_hf_config_read(argv[i], &c);
    } else if (mode == "safetensors") {
      rc = safetensors(argv[i]);
    } else if (mode == "eos") {
      size_t n = 0;
      uint32_t ids[64];
      rc = llrs_find_eos_tokens(argv[i], ids, 64, &n);
    } else if (mode == "quantize") {
      rc = quantize(argv[i]);
    } else {
      fprintf(stderr, "unknown mode %s\n", mode.c_str());
      return 2;
    }
    report(argv[i], rc);
  }
  return 0;
}
