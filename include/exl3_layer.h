/*
 * exl3_layer.h — C-ABI of the MI355X (gfx950) kernels of the layer pipeline
 * around the trellis encoder (alpha2beta/EXL3_Intel_Arc_quantizer's
 * exl3_quant/hadamard.py, regularize.py and ldlq.py, which do this work with
 * torch tensor operations). Same conventions as exl3_encoder.h: device
 * buffers owned by the caller, nothing allocated, work enqueued on `stream`
 * (a hipStream_t, NULL = the null stream), 0 on success and a message in
 * exl3_last_error() otherwise. Matrices are float32, row-major, contiguous.
 */
#ifndef EXL3_LAYER_H
#define EXL3_LAYER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces preapply_had_l / preapply_had_r (hadamard.py:73-96) and their
 * in-place forms (hadamard.py:99-126): the orthonormal Sylvester matrix of
 * order 128, H[i][j] = (-1)^popcount(i & j) / sqrt(128), applied blockwise.
 * side = 0: out = H @ in on every 128-row block (rows % 128 == 0);
 * side = 1: out = in @ H on every 128-column block (cols % 128 == 0).
 * Computed as a fast Walsh-Hadamard transform in fp32; in == out is allowed. */
int exl3_hadamard128(const float* in, float* out, int64_t rows, int64_t cols, int side,
                     void* stream);

/* The two fused steps of regularize (regularize.py:171-181): each divides
 * the matrix by a scale vector and applies the blockwise Hadamard transform
 * in one pass over HBM, the arithmetic of a division (correctly rounded
 * fp32) followed by exl3_hadamard128.
 * side = 1: out = (in / divisor[col]) @ H, divisor of `cols` floats (the
 *           fold of sv before H_r); slice_sumsq, if not NULL, receives the
 *           sum of squares of every 32-element slice of every output row,
 *           slice_sumsq[row * (cols / 32) + slice] (the first pass of the
 *           row RMS that regularize takes next).
 * side = 0: out = H @ (in / divisor[row]), divisor of `rows` floats (the
 *           fold of su before H_l); slice_sumsq must be NULL.
 * divisor may be NULL (no division); in == out is allowed. */
int exl3_hadamard128_scaled(const float* in, float* out, int64_t rows, int64_t cols, int side,
                            const float* divisor, float* slice_sumsq, void* stream);

/* Second pass of block_rms (regularize.py:41-56) over slice sums made
 * elsewhere: out[o] = sqrt(S_o / n), S_o the sum of slice_sumsq[o * slices
 * + s] over s = 0 .. slices - 1 taken in slice order. */
int exl3_block_rms_from_slices(const float* slice_sumsq, float* out, int64_t outputs, int64_t n,
                               int64_t slices, void* stream);

/* Replaces block_rms (regularize.py:41-56): out = sqrt(S / n), S the sum of
 * squares along `dim` (0: over rows, one output per column; 1: over
 * columns, one per row) taken in slices of `blocksize` whose sums are
 * accumulated in slice order. workspace: device floats, at least
 * exl3_block_rms_workspace(rows, cols, dim, blocksize) of them (the slice
 * sums). */
int exl3_block_rms(const float* x, float* out, int64_t rows, int64_t cols, int dim, int blocksize,
                   float* workspace, int64_t workspace_elems, void* stream);

/* Floats of workspace exl3_block_rms needs (outputs x slices), or -1 for
 * invalid arguments. */
int64_t exl3_block_rms_workspace(int64_t rows, int64_t cols, int dim, int blocksize);

/* The diagonal-block step of a blocked Cholesky factorisation, which
 * replaces torch.linalg.cholesky_ex in block_ldl (ldlq.py:76-142): factors
 * the nb x nb block at `a` (leading dimension lda, lower triangle read,
 * nb <= exl3_cholesky_block_order()) in place into L (zeros above the
 * diagonal). A non-positive or NaN pivot k sets *info (device int32) to
 * offset + k + 1 unless it is already non-zero. */
int exl3_cholesky_diag_block(float* a, int64_t lda, int nb, int64_t offset, int32_t* info,
                             void* stream);

/* Largest block order exl3_cholesky_diag_block accepts (128). */
int exl3_cholesky_block_order(void);

/* One 16-row block of an LDLQ traversal inside an encoder call: device
 * addresses (as integers) of the block's first row in W, in its
 * compensation rows, in Wq and in E = W - Wq (all float, row stride n), of
 * its (n / 16, 256) int16 states, and the block's first tile in the call's
 * batch. A call's blocks are listed in batch order, back to back
 * (tile0 of block b + 1 = tile0 + n / 16 of block b). The table itself is
 * read by the kernels, so it lives in device memory. */
typedef struct exl3_ldlq_block {
  int64_t w;
  int64_t comp;
  int64_t wq;
  int64_t err;
  int64_t states;
  int64_t n;
  int64_t tile0;
  int64_t reserved;
} exl3_ldlq_block;

/* Replaces the tile formation of one LDLQ step (ldlq.py:276-287) for every
 * block of an encoder call: x[tile0 + t][p] = W[r][16 t + c] + comp[r][16 t + c]
 * with (r, c) the row and column of tensor_core_perm(p) in a 16 x 16 tile.
 * x is f32 [tiles][256]; tiles = the sum of the blocks' n / 16. */
int exl3_ldlq_gather(const exl3_ldlq_block* blocks, int nblocks, int64_t tiles, float* x,
                     void* stream);

/* Replaces the write-back of one LDLQ step (ldlq.py:289-300) for every
 * block of an encoder call, from the encoder's tensor-core-order outputs
 * recon (f32 [tiles][256]) and idx (int16 [tiles][256]): Wq[r][16 t + c] =
 * recon, E[r][16 t + c] = W - recon at the same position, and the block's
 * states[t][p] = idx[tile0 + t][p]. */
int exl3_ldlq_scatter(const exl3_ldlq_block* blocks, int nblocks, int64_t tiles,
                      const float* recon, const int16_t* idx, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_LAYER_H */
