// On-device sampling of the next token from the current logits
// (InferenceEngine::sample_current_logits, src/engine.rs:253-325).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace llrs {

struct SampleParams {
  float temperature;  // <= 0: the first of the sorted candidates (greedy)
  int top_k;          // 0: every token
  float top_p;        // in (0, 1]
  float penalty;      // repetition penalty; 1: off
};

// Device scratch for a vocabulary of n tokens: sort keys and indices (in and
// out), the radix sort's temporary storage, the repeat window, the result.
struct SampleScratch {
  int n = 0, max_recent = 0;
  uint32_t *keys = nullptr, *keys_sorted = nullptr, *idx = nullptr, *idx_sorted = nullptr;
  uint32_t *recent = nullptr, *token = nullptr;
  void *tmp = nullptr;
  size_t tmp_bytes = 0;
};

// Temporary bytes of the descending radix sort of n (key, index) pairs.
size_t sample_sort_bytes(int n);

// Limits of the allocation-free sampler: vocabulary, repeat window, and the
// bytes reserved for the radix sort's temporary storage.
constexpr int kNoAllocMaxVocab = 262144;
constexpr int kNoAllocMaxRecent = 65536;
constexpr size_t kNoAllocSortBytes = 4u << 20;

// Points w into this device's file-scope scratch array (the current device's
// copy, looked up once per device with hipGetSymbolAddress): no allocation.
// Fails if the radix sort of kNoAllocMaxVocab pairs needs more temporary
// storage than kNoAllocSortBytes.  Every call on one device shares the array.
int sample_noalloc_scratch(SampleScratch &w);

// Samples from logits[0, n) into *w.token (device), using the uniform draw u
// in [0, 1); recent[0, n_recent) is already on the device (w.recent).
int launch_sample(const float *logits, int n, const SampleParams &p, int n_recent, float u,
                  SampleScratch &w, hipStream_t s);

}  // namespace llrs
