/*
 * CPU restatement of hachiue's lm_head GEMV (the logits producer before the
 * sampler): output.weight [N rows x K] in a GGML block format times the
 * final hidden state x [M x K], y[m][n] = sum_k x[m][k] * W[n][k].
 *
 * TEST INFRASTRUCTURE ONLY, like sampler_oracle.h: only tests, the smoke
 * check and the CPU-baseline leg of the benchmark may load it.
 *
 * Formats: those the reference uploads as raw GGML blocks
 * (src/engine.ts:772-800): F32, Q4_0, Q4_1, Q4_K, Q6_K; and the 128-weight
 * binary / ternary formats Q1_0, PQ2_0, PTQ1_0 (src/gguf.ts:56-63, decoded
 * by src/gguf.ts:93-147), given here in their GGUF block form.  A row of W is
 * K / B consecutive blocks of the format (B weights per block), rows back to
 * back.
 */
#ifndef HACHIUE_LMHEAD_ORACLE_H
#define HACHIUE_LMHEAD_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (src/types.ts:4-15). */
enum { ORC_W_F32 = 0, ORC_W_Q4_0 = 2, ORC_W_Q4_1 = 3, ORC_W_Q4_K = 12, ORC_W_Q6_K = 14,
       ORC_W_Q1_0 = 41, ORC_W_PQ2_0 = 142, ORC_W_PTQ1_0 = 143 };

/* Weights per block and bytes per block (src/gguf.ts getBlockSpec); 0 for an
 * unknown type. */
int orc_block_weights(int type);
int orc_block_bytes(int type);

/* IEEE binary16 to binary32 (src/gguf.ts:81-88). */
float orc_fp16(uint16_t h);

/* One row of W (K weights, K a multiple of the block size) dequantised as
 * src/gguf.ts:149-230 (dequantizeBlockCpu) and src/gguf.ts:93-147
 * (dequantizeBlock128Cpu) do, in binary32. */
int orc_dequant_row(int type, const uint8_t *row, int64_t K, float *out);

/* y = x W^T with every product and sum in binary64 from the dequantised
 * binary32 weights: the value the GEMV approximates.  Also writes
 * mag[m][n] = sum_k |x[m][k] * W[n][k]| (may be NULL), which bounds the
 * rounding error of any binary32 summation order. */
int orc_gemv_exact(int type, const float *x, int64_t M, int64_t K, const uint8_t *w,
                   int64_t N, double *y, double *mag);

/* The reference's own binary32 result, step by step in its order
 * (src/kernels.ts:244-290 gemv_f32, :717-800 gemv_q4_0, :807-888 gemv_q4_1,
 * :896-997 gemv_q4_k, :1003-1090 gemv_q6_k): 64 invocations per row, each
 * accumulating its blocks (or 32-weight units) in turn, then a shared-memory
 * tree (stride 32 down to 1).  Products and sums are rounded to binary32 one
 * at a time (no fused multiply-add).  Not defined for Q1_0, PQ2_0, PTQ1_0
 * (returns -1): their WGSL kernels sum through vec4 dot(), whose order WGSL
 * leaves open. */
int orc_gemv_ref(int type, const float *x, int64_t M, int64_t K, const uint8_t *w, int64_t N,
                 float *y);

/* The 512-wide Walsh-Hadamard rotation of a hadamard-folded weight's input
 * (src/kernels.ts:177-227 hadamard_512, mode 0, as src/engine.ts:1121-1145
 * runs it before the GEMV): for each of `rows` rows of `width` binary32
 * values (width a multiple of 512), each 512-block is multiplied by
 * signs[col] (when signs is not NULL), goes through the nine butterfly
 * stages (a + b, a - b in binary32) and is scaled by binary32(1/sqrt(512)).
 * In place. */
int orc_hadamard512(float *x, int64_t rows, int64_t width, const float *signs);

#ifdef __cplusplus
}
#endif

#endif
