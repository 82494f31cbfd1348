// Kernel argument block of the FlashAttention kernels (flash_fwd.hip,
// flash_f32.hip); must match struct FlashParams in capi/ops_attn.cpp.
#pragma once

struct FlashParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;  // [B, H, S] or null
  long long sqb, sqh, sqs;
  long long skb, skh, sks;
  long long svb, svh, svs;
  long long sob, soh, sos;
  int B, H, S, D;
  float sl2;  // softmax scale * log2(e)
  int causal;
  int dtype;  // general kernel only
};
