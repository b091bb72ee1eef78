/*
 * fa_oracle.h — TEST INFRASTRUCTURE ONLY. CPU restatement of ggml's
 * GGML_OP_FLASH_ATTN_EXT, used as the parity checker for the HIP path and
 * as the CPU baseline timed by bench.py. Nothing in the product links it.
 *
 * Tensors use the same descriptor as the C ABI (include/vxfa.h), but `data`
 * points to HOST memory here.
 */
#ifndef FA_ORACLE_H
#define FA_ORACLE_H

#include <stdint.h>
#include "../include/vxfa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE-754 binary16 <-> binary32, round-to-nearest-even. */
float    oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void     oracle_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n);
void     oracle_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n);

/* Flags for oracle_fa_ggml. */
enum {
    ORACLE_VKQ_F16 = 1,   /* accumulate V*softmax in f16 when V is f16 (ggml's one-row CPU kernel) */
    /* Deliberate mistakes, used only by tests to show that the checks catch them. */
    ORACLE_MUT_GQA_MOD   = 1 << 8,  /* kv head = h % Hkv instead of h / (Hq/Hkv) */
    ORACLE_MUT_NO_MASK   = 1 << 9,  /* ignore the mask */
    ORACLE_MUT_NO_SCALE  = 1 << 10, /* forget the scale */
    ORACLE_MUT_V_SHIFT   = 1 << 11, /* read V one position late */
    ORACLE_MUT_NO_MAXSUB = 1 << 12, /* skip the running-max rescale of the sum */
};

/* ggml-faithful one-row algorithm (per query row, per head, per batch):
 * Q converted to K's dot type (f16 for f16 K), masked (-inf) positions
 * skipped, online softmax with expf, V accumulated in f16 or f32, output
 * scaled by 1/S (0 when S == 0), written in the permuted dst layout.
 * Threads: rows are split across n_threads (<= 0 means 1).
 * max_bias and logit_softcap must be 0 (voxtral's arguments; ALiBi and
 * soft-capping are not restated). Returns 0, or -1 on a contract violation
 * or a nonzero max_bias / logit_softcap. */
int oracle_fa_ggml(const vxfa_tensor* q, const vxfa_tensor* k,
                   const vxfa_tensor* v, const vxfa_tensor* mask,
                   vxfa_tensor* dst, float scale, float max_bias,
                   float logit_softcap, int flags, int n_threads);

/* Exact reference in double precision: two-pass softmax over the unmasked
 * positions. q_f16 != 0 rounds Q to f16 first (as ggml does for f16 K).
 * Fully masked rows give zeros. dst is double [D, Hq, Nq, B] contiguous.
 * max_bias and logit_softcap must be 0, as above. */
int oracle_fa_f64(const vxfa_tensor* q, const vxfa_tensor* k,
                  const vxfa_tensor* v, const vxfa_tensor* mask,
                  double* dst, float scale, float max_bias,
                  float logit_softcap, int q_f16, int n_threads);

/* The same one-row algorithm with ggml-cpu's AVX2 / F16C vector kernels
 * (fa_cpu_simd.c): the CPU baseline bench.py times. F16 K and V, F32 or F16
 * Q, optional F16 mask; V accumulated in f16 as ggml's one-row kernel does.
 * Returns 0, or -1 on a contract violation. */
int oracle_fa_cpu_simd(const vxfa_tensor* q, const vxfa_tensor* k,
                       const vxfa_tensor* v, const vxfa_tensor* mask,
                       vxfa_tensor* dst, float scale, int n_threads);

#ifdef __cplusplus
}
#endif

#endif
