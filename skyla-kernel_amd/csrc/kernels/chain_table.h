// Stage table of matvec_chain (chain.hip), written by the host runtime (skyla_hip.cpp) and
// read by the kernel with scalar loads.  Plain data, the same layout on both sides.
#pragma once

#include <stdint.h>

// Stage kinds: the dense decode matvec shapes the chain computes.
enum : uint32_t {
  CHAIN_Q4K_4096 = 1,   // Q4_K, n_in = 4096, chunks of 8 rows
  CHAIN_Q6K_12288 = 2,  // Q6_K, n_in = 12288, chunks of 2 rows
};

// One segment of a stage (one engine dispatch of a fused launch).
struct ChainSeg {
  uint32_t o[4];   // region offsets in units of 16 B (Q6_K d: units of 2 B), as the push words
  uint32_t n_out;  // rows
  uint32_t y_off;  // f32 offset of row 0's output in the output buffer
  uint32_t g_end;  // chunks of the stage up to and including this segment (~0 past n_seg)
  uint32_t pad;
};

struct ChainStage {
  uint64_t w, x, y;    // device addresses: weights, activations, outputs
  uint32_t kind;       // CHAIN_*
  uint32_t accum;      // 1: y += W x
  uint32_t n_seg;      // 1..4
  uint32_t n_chunks;   // chunks (row groups) of the stage
  uint32_t x_off;      // f32 offset of the activations in x
  uint32_t w_records;  // bytes of w the stage may read (loads past it return zero)
  uint32_t pad[4];
  ChainSeg seg[4];
};

static_assert(sizeof(ChainSeg) == 32, "ChainSeg layout");
static_assert(sizeof(ChainStage) == 192, "ChainStage layout");

// Grid of matvec_chain: one workgroup per CU, CHAIN_THREADS threads each.
#define CHAIN_THREADS 640
// Words of the chain's synchronisation area: [0] barrier arrivals, [1] time-out flag.
#define CHAIN_SYNC_WORDS 2
