/*
 * skyla_oracle.h -- CPU restatement of the reference's f32 path
 * (skyla-gguf/src/quant.rs, skyla-gguf/src/lib.rs, skyla-ref/src/{matrix,ffn,ops}.rs,
 * skyla-shaders/shaders/moe_sort.comp).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the correctness checker for the HIP path
 * and the reported CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library (libskyla_hip.so) never links,
 * loads or calls it.
 *
 * Built with -O2 -ffp-contract=off and no -march=native (oracle/Makefile): Rust never
 * contracts a*b+c into an FMA, so neither may this restatement.
 *
 * Every function returns 0 on success and a negative SK_E* code on bad input, the C
 * restatement of the reference's anyhow::bail!/ensure! paths.
 */
#ifndef SKYLA_ORACLE_H
#define SKYLA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (skyla-gguf/src/lib.rs:23-31) */
#define SK_F32 0u
#define SK_F16 1u
#define SK_Q8_0 8u
#define SK_Q4K 12u
#define SK_Q6K 14u

#define SK_OK 0
#define SK_E_TYPE (-1)     /* "unsupported ggml type" (skyla-gguf/src/lib.rs:41) */
#define SK_E_ROW (-2)      /* "row of n elements is not a multiple of .." (lib.rs:47-50) */
#define SK_E_SIZE (-3)     /* slice length mismatch (matrix.rs:44 assert_eq) */
#define SK_E_THREAD (-4)   /* thread spawn failed */

/* half 2.7.1 f16::to_f32 / f16::from_f32 (Cargo.lock:58-59), IEEE-754 binary16. */
float sk_f16_to_f32(uint16_t h);
uint16_t sk_f32_to_f16(float f);

/* DType::block / DType::row_bytes (skyla-gguf/src/lib.rs:33-53). */
int sk_block(uint32_t type, uint64_t *per_block, uint64_t *bytes);
int64_t sk_row_bytes(uint32_t type, uint64_t n);

/* quant.rs:5-38 dequantize; quant.rs:40-49 q4k_scale_min; quant.rs:91-101 quantize_q8_0 */
int sk_dequantize(uint32_t type, const uint8_t *src, uint64_t src_len, float *out, uint64_t out_len);
void sk_q4k_scale_min(uint32_t j, const uint8_t *scales, uint8_t *sc, uint8_t *m);
void sk_quantize_q8_0(const float *src, uint64_t n, uint8_t *out);

/* Matrix::matvec (skyla-ref/src/matrix.rs:43-58).  threads == 0 means
 * available_parallelism(); the result does not depend on the thread count. */
int sk_matvec(uint32_t type, const uint8_t *data, uint64_t n_in, uint64_t n_out,
              const float *x, float *y, uint32_t threads);
/* The oracle's f32 GEMM: n_tok independent Matrix::matvec calls, token-major
 * x[tok * x_stride + k] and y[tok * y_stride + row]. */
int sk_matmul(uint32_t type, const uint8_t *data, uint64_t n_in, uint64_t n_out,
              uint64_t n_tok, const float *x, uint64_t x_stride, float *y, uint64_t y_stride,
              uint32_t threads);

/* ops.rs */
void sk_rmsnorm(const float *x, const float *w, uint64_t n, float eps, float *out);
void sk_softmax(float *x, uint64_t n);
float sk_silu(float x);
float sk_dot(const float *a, const float *b, uint64_t n);
uint32_t sk_argmax(const float *x, uint64_t n);

/* ffn.rs:30-37 route: ids/weights receive `used` entries. */
int sk_route(const float *router, const float *n, uint64_t n_embd, uint64_t n_expert,
             uint64_t used, uint32_t *ids, float *weights);
/* ffn.rs:21-28 swiglu(gate, up, down, n, out). */
int sk_swiglu(uint32_t gate_type, const uint8_t *gate, uint32_t up_type, const uint8_t *up,
              uint32_t down_type, const uint8_t *down, uint64_t n_embd, uint64_t n_ff,
              const float *n, float *out, uint32_t threads);
/* ffn.rs:58-76 Ffn::forward, Moe arm: experts stacked [n_expert][n_out][row_bytes]
 * (matrix.rs:30-36).  ids/weights (may be NULL) receive the route. */
int sk_moe_forward(const float *router, uint32_t gate_type, const uint8_t *gate_exps,
                   uint32_t up_type, const uint8_t *up_exps, uint32_t down_type,
                   const uint8_t *down_exps, uint64_t n_embd, uint64_t n_ff, uint64_t n_expert,
                   uint64_t used, const float *n, float *out, uint32_t *ids, float *weights,
                   uint32_t threads);
/* moe_sort.comp:21-55: table[2e] = count, table[2e+1] = start; list[start + rank] = slot
 * with rank = number of earlier slots routed to the same expert (stable). */
int sk_moe_sort(const uint32_t *ids, uint64_t n_slots, uint32_t n_expert, uint32_t *table,
                uint32_t *list);

uint32_t sk_available_parallelism(void);

/* The rest of the dense decode step (skyla-ref/src/ops.rs, rope.rs, model.rs:131-170). */
void sk_rmsnorm_inplace(float *x, const float *w, uint64_t n, float eps);
void sk_rope_freqs(uint64_t head_dim, float theta, float *out);
float sk_rope_freqs_yarn(uint64_t head_dim, float theta, float factor, float original_ctx, float attn_factor,
                         float *out);
void sk_rope_neox(float *x, uint64_t n, uint64_t pos, const float *freqs, float mscale);
void sk_attention(const float *q, const float *k_cache, const float *v_cache, uint64_t n_pos,
                  uint64_t n_head, uint64_t n_head_kv, uint64_t hd, float *scores, float *out);

#ifdef __cplusplus
}
#endif
#endif
