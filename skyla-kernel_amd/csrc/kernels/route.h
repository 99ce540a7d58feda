// moe_route's selection and routing weights, shared by moe.hip (moe_route) and matvec.hip
// (the experts' gate/up form that routes for itself).
#pragma once

#include "common.h"

struct RoutePush { uint32_t logits_off, ids_off, weights_off, n_expert, n_used; };

// Monotone u32 key of a float with -0 folded onto +0 (so equal values tie exactly as the
// float comparisons of moe_route.comp:36-52 do).
SK_DEV uint32_t order_key(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

SK_DEV float key_value(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __builtin_bit_cast(float, b);
}

// moe_route's selection (moe_route.comp:23-74): n_used rounds of "largest logit, lowest
// index on ties" give the same experts, in the same order, as ranking every expert: expert
// e's place is the number of experts before it in the order "larger key first, lower index
// on ties" (all (key, index) pairs are distinct, so the places are 0, 1, ..), and the
// expert in place k is round k's choice.  One workgroup of 256 threads per token: each
// (key, ~index) pair is one 64-bit word in LDS, and thread t counts the words above expert
// t % 128's over half of the experts (n_expert <= 128) or expert t's over all of them, with
// no serial rounds.  Leaves sid[k] = the expert in place k and sval[k] = its logit (read
// back from the key, -0 as +0) for k < n_used, behind a barrier.  Needs n_used <= n_expert
// (the engine's configuration check).
SK_DEV void route_ranked(const float *a, const RoutePush &p, uint32_t tok, uint32_t t, uint32_t *sid,
                         float *sval) {
  __shared__ uint64_t kk[256];
  __shared__ uint32_t half[256];
  const uint32_t n_used = min(p.n_used, 16u);
  const uint32_t n_expert = min(p.n_expert, 256u);
  uint32_t key = 0;
  if (t < n_expert) key = max(order_key(a[p.logits_off + tok * p.n_expert + t]), 1u);
  kk[t] = ((uint64_t)key << 32) | (uint32_t)~t;
  __syncthreads();
  const bool halves = n_expert <= 128;  // wave-uniform: waves 0, 1 take the first half
  const uint32_t e = halves ? (t & 127) : t;
  const uint32_t len = halves ? (n_expert + 1) / 2 : n_expert;
  const uint32_t f0 = halves ? (t >> 7) * len : 0, f1 = min(f0 + len, n_expert);
  const uint64_t mine = kk[e];
  uint32_t before = 0;
#pragma unroll 8
  for (uint32_t f = f0; f < f1; f++) before += kk[f] > mine ? 1u : 0u;
  half[t] = before;
  __syncthreads();
  if (t < n_expert) {  // with halves, t < 128: thread t + 128 counted the second half
    const uint32_t place = before + (halves ? half[t + 128] : 0u);
    if (place < n_used) {
      sid[place] = t;
      sval[place] = key_value(key);
    }
  }
  __syncthreads();
}

// The routing weight of lane t's choice `chosen` (lane k holds place k's logit, for the first
// 64 lanes of the workgroup): exp(v_k - v_0) over the sum of the n_used exponentials, added in
// place order (moe_route.comp:66-73).
SK_DEV float route_weight(float chosen, uint32_t n_used) {
  const float largest = __shfl(chosen, 0, 64);
  const float e = expf(chosen - largest);
  float total = 0.0f;
  for (uint32_t k = 0; k < n_used; k++) total += __shfl(e, (int)k, 64);
  return e / total;
}
