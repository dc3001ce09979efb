/* oracle/knj_oracle.h -- CPU oracle for the MoE decode path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product: only tests/, the smoke() entry
 * point and the bench's CPU-baseline leg load it.  It restates the reference's CPU
 * forward pass (/root/reference/src/model/model.cpp, src/loader/dequant.cpp) in
 * the reference's own order of floating-point operations, so the GPU path is
 * graded against what Kanjoos itself computes.
 *
 * Deliberate differences from the reference, each required by the benchmark
 * configurations:
 *   - weights come from an in-memory image (include/knj_model.h), not a GGUF
 *     mapping (the reference's mapping is Windows-only, gguf.cpp:405-406);
 *   - the KV cache is f16 (round-to-nearest-even) instead of f32.
 */
#ifndef KNJ_ORACLE_H
#define KNJ_ORACLE_H

#include <stdint.h>

#include "../include/knj_model.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- format primitives (dequant.cpp:1032-1112) ---- */
float knjo_f16_to_f32(uint16_t h);
uint16_t knjo_f32_to_f16(float f);
float knjo_bf16_to_f32(uint16_t b);
void knjo_dequant_row_f32(int type, const uint8_t* src, float* dst, uint64_t n);
float knjo_dequant_dot_f32(int type, const uint8_t* src, const float* x, uint64_t n);

/* ---- synthetic tensors (include/knj_synth.h), threaded ---- */
/* n_rows rows of n_in weights of `type`, element (r, i) = N(0, std) of index r*n_in+i. */
void knjo_synth_tensor(uint64_t key, int type, uint64_t n_in, uint64_t n_rows, float stddev,
                       uint8_t* out, int threads);
uint64_t knjo_tensor_key(uint64_t seed, int layer, int kind, int expert);
/* Fill a whole weight image (knj_model_layout) for cfg/seed. */
void knjo_synth_model(const knj_model_config* cfg, uint64_t seed, uint8_t* image, int threads);

/* ---- GEMV (Model::matmul, model.cpp:326-380, m rows of x) ---- */
void knjo_matmul(int type, const uint8_t* w, int n_in, int n_out, const float* x, int m,
                 float* y, int threads);

/* ---- router + MoE FFN (Model::moe, model.cpp:399-510) ----
 * hx: m rows of n_embd (already RMS-normalised).  gate/up/down point at the
 * [n_expert] slabs.  Outputs: out [m][n_embd], logits [m][n_expert],
 * topk_idx / topk_w [m][k] in selection order. */
void knjo_moe(const float* hx, int m, int n_embd, int n_ff, int n_expert, int k,
              const float* router_w, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
              int type_gate_up, int type_down, float* out, float* logits, int32_t* topk_idx,
              float* topk_w, int threads);

/* ---- RMSNorm (model.cpp:240-271) ---- */
void knjo_rmsnorm(const float* x, const float* w, float* out, int width, float eps);

/* ---- model (Model::open/forward/reset, model.cpp:174-238, 512-672) ---- */
typedef struct knjo_model knjo_model;
/* Builds the synthetic weights itself when `image` is NULL; otherwise uses (does
 * not copy) the caller's image, which must outlive the model. */
knjo_model* knjo_model_create(const knj_model_config* cfg, uint64_t seed, const uint8_t* image,
                              int threads);
void knjo_model_free(knjo_model* m);
const uint8_t* knjo_model_image(knjo_model* m);
uint64_t knjo_model_image_bytes(knjo_model* m);
void knjo_model_reset(knjo_model* m);
int knjo_model_pos(knjo_model* m);
int knjo_model_threads(knjo_model* m);
/* Runs n tokens as one Model::forward call (all rows through each weight, all
 * keys appended, causal attention); copies the last token's logits into
 * `logits` (n_vocab floats).  Returns 0, or -1 with a message in
 * knjo_last_error(). */
int knjo_model_forward(knjo_model* m, const int32_t* tokens, int n, float* logits);
/* The same n tokens as n single-token forward calls (identical for n == 1). */
int knjo_model_forward_steps(knjo_model* m, const int32_t* tokens, int n, float* logits);
/* Residual stream of the last token after layer il (model.cpp:654-658), from
 * the most recent forward call. */
const float* knjo_model_hidden(knjo_model* m, int il);
/* Router choices of the last token in layer il: k indices then k weights. */
const int32_t* knjo_model_topk_idx(knjo_model* m, int il);
const float* knjo_model_topk_w(knjo_model* m, int il);
/* The f16 KV cache (layout in knj_model.h) and the position setter used to
 * continue from a cache filled elsewhere. */
uint16_t* knjo_model_kv_k(knjo_model* m);
uint16_t* knjo_model_kv_v(knjo_model* m);
int knjo_model_set_pos(knjo_model* m, int pos);
/* Cache-source mode: when k/v are non-NULL (same layout as the model's cache),
 * each newly written cache element takes the source's f16 value.  Statistics
 * since the last call: elements adopted, elements that differed from the
 * oracle's own rounding, the largest difference in f16 ulps, and the largest
 * absolute distance from the oracle's f32 value to the set of f32 values that
 * round to the source's f16 value (K and V elements are O(1) here, so a bound
 * like 1e-5 says the source rounded an f32 value that agrees with the oracle's
 * to ~1e-5 relative). */
void knjo_model_set_kv_source(knjo_model* m, const uint16_t* k, const uint16_t* v);
void knjo_model_kv_stats(knjo_model* m, int64_t* adopted, int64_t* differing, int* max_ulp,
                         float* max_mid_dist);
/* Sums over the adopted elements since knjo_model_set_kv_source: squared
 * distance to the rounding interval of the adopted value, squared own value;
 * sqrt(d2 / v2) is the relative RMS distance of the adopted cache writes. */
void knjo_model_kv_rms(knjo_model* m, double* sum_d2, double* sum_v2);
const char* knjo_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KNJ_ORACLE_H */
