// MI355X (gfx950) kernels of the layer pipeline around the trellis encoder
// (reference: exl3_quant/hadamard.py, regularize.py, ldlq.py):
//
//   had128_right_kernel / had128_left_kernel
//       the blockwise orthonormal Sylvester transform of order 128 as a fast
//       Walsh-Hadamard transform: 7 butterfly levels of fp32 add/sub and one
//       scale instead of a 128-term dot product per output. HBM-bound: one
//       read and one write of the matrix. Right (x @ H per 128-column
//       block): one wave per 128-element row segment, two elements per lane,
//       levels 2..7 across lanes. Left (H @ x per 128-row block): one thread
//       per column of a row block, the 128 values in registers; loads and
//       stores are coalesced across the wave's 64 columns.
//   block_rms_slices_kernel / block_rms_reduce_kernel
//       sqrt(sum of squares / n) along one dimension: one thread per slice
//       of `blocksize` sums its squares in order, then one thread per output
//       accumulates the slice sums in slice order.
//   cholesky_diag_kernel
//       the unblocked Cholesky factorisation of one diagonal block (order
//       <= 128) inside a blocked factorisation whose panel updates and
//       triangular solves are GEMM-class library calls: 256 threads each
//       hold an 8x8 sub-block of the lower triangle in registers; column k
//       is published through a double-buffered LDS vector, one barrier per
//       column.
//   ldlq_gather_kernel / ldlq_scatter_kernel
//       one LDLQ step's tile formation and write-back for every 16-row block
//       of an encoder call, one 256-thread workgroup per tile: thread p moves
//       tensor-core element p between the tile and row r, column 16 t + c of
//       the block (W + compensation in; Wq, E = W - Wq and the states out).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/exl3_layer.h"
#include "exl3_errors.h"
#include "exl3_layout.h"

using exl3::check_launch;
using exl3::set_error;

namespace {

// 1 / sqrt(128), rounded to fp32.
constexpr float kHadScale = 0.088388347648318440550f;

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------- Hadamard

constexpr int HAD_N = 128;
constexpr int HAD_RIGHT_WAVES = 4;

// Butterfly of lane distance h: the lane without bit h holds the lower
// element a of each pair (a, b) and keeps a + b, its partner keeps a - b.
__device__ __forceinline__ float had_level(float v, int lane, int h) {
  const float p = __shfl_xor(v, h, 64);
  return (lane & h) ? p - v : v + p;
}

// DIV: every element of column c is divided by div[c] before the transform
// (regularize's fold of sv into the weight). SUMSQ: the sum of squares of
// each 32-element slice of the transformed row goes to
// sumsq[row * (cols / 32) + slice] (the first pass of the row RMS that
// follows the transform); lanes 16 j .. 16 j + 15 hold slice j of the
// segment and add their squares in a butterfly.
template <bool DIV, bool SUMSQ>
__global__ void __launch_bounds__(64 * HAD_RIGHT_WAVES)
    had128_right_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t segments,
                        int64_t seg_per_row, const float* __restrict__ div,
                        float* __restrict__ sumsq) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * HAD_RIGHT_WAVES;
  for (int64_t seg = (int64_t)blockIdx.x * HAD_RIGHT_WAVES + (threadIdx.x >> 6); seg < segments;
       seg += stride) {
    // Lane l holds elements 2l and 2l + 1 of the segment.
    float2 v = reinterpret_cast<const float2*>(in + seg * HAD_N)[lane];
    if (DIV) {
      const float2 d =
          reinterpret_cast<const float2*>(div + (seg % seg_per_row) * HAD_N)[lane];
      v.x = v.x / d.x;
      v.y = v.y / d.y;
    }
    float lo = v.x + v.y, hi = v.x - v.y;
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
      lo = had_level(lo, lane, h);
      hi = had_level(hi, lane, h);
    }
    lo = lo * kHadScale;
    hi = hi * kHadScale;
    reinterpret_cast<float2*>(out + seg * HAD_N)[lane] = make_float2(lo, hi);
    if (SUMSQ) {
      float q = lo * lo + hi * hi;
#pragma unroll
      for (int h = 1; h < 16; h <<= 1) q = q + __shfl_xor(q, h, 64);
      if ((lane & 15) == 0) sumsq[seg * (HAD_N / 32) + (lane >> 4)] = q;
    }
  }
}

// DIV: every element of row r is divided by div[r] before the transform
// (the fold of su).
template <bool DIV>
__global__ void __launch_bounds__(256)
    had128_left_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t cols,
                       const float* __restrict__ div) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  const int64_t row0 = (int64_t)blockIdx.y * HAD_N;
  const int64_t base = row0 * cols + c;
  float v[HAD_N];
#pragma unroll
  for (int r = 0; r < HAD_N; ++r) {
    v[r] = in[base + r * cols];
    if (DIV) v[r] = v[r] / div[row0 + r];
  }
#pragma unroll
  for (int h = 1; h < HAD_N; h <<= 1) {
#pragma unroll
    for (int i = 0; i < HAD_N; ++i) {
      if (!(i & h)) {
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < HAD_N; ++r) out[base + r * cols] = v[r] * kHadScale;
}

// --------------------------------------------------------------- block RMS

// Output o reduces x[o * so + t * st] over t < n, in ns slices of bs.
// Pass 1: one thread per (output, slice) sums the slice's squares in order
// into ws: slice-major (ws[s * outputs + o]) when dim = 0, so that threads
// of a wave read adjacent columns, output-major (ws[o * ns + s]) when
// dim = 1, so that they read adjacent slices of one row.
__global__ void __launch_bounds__(256)
    block_rms_slices_kernel(const float* __restrict__ x, float* __restrict__ ws, int64_t outputs,
                            int64_t n, int64_t so, int64_t st, int bs, int64_t ns, int dim) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= outputs * ns) return;
  const int64_t o = dim == 0 ? idx % outputs : idx / ns;
  const int64_t s = dim == 0 ? idx / outputs : idx % ns;
  const int64_t t0 = s * bs, t1 = t0 + bs < n ? t0 + bs : n;
  const float* p = x + o * so;
  float slice = 0.0f;
  for (int64_t t = t0; t < t1; ++t) {
    const float v = p[t * st];
    const float sq = v * v;
    slice = slice + sq;
  }
  ws[idx] = slice;
}

// Pass 2: one thread per output accumulates its slice sums in slice order.
__global__ void __launch_bounds__(256)
    block_rms_reduce_kernel(const float* __restrict__ ws, float* __restrict__ out,
                            int64_t outputs, int64_t n, int64_t ns, int dim) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= outputs) return;
  float acc = 0.0f;
  for (int64_t s = 0; s < ns; ++s) {
    const float v = dim == 0 ? ws[s * outputs + o] : ws[o * ns + s];
    acc = (s == 0) ? v : acc + v;
  }
  out[o] = sqrtf(acc / (float)n);
}

// -------------------------------------------------------- Cholesky block

constexpr int CH_NB = 128;              // largest block order
constexpr int CH_SB = 8;                // rows / columns of a thread's sub-block
constexpr int CH_GRID = CH_NB / CH_SB;  // 16 x 16 sub-blocks
constexpr int CH_THREADS = CH_GRID * CH_GRID;

// Factors the nb x nb block at `a` (row-major, leading dimension lda,
// lower triangle read) in place: L on and below the diagonal, zeros above.
// Positions past nb act as an identity block and are never stored. A pivot
// that is not positive (or NaN) sets *info to offset + k + 1 if *info is
// still 0; the factorisation then carries on and its result is meaningless,
// as LAPACK's potrf leaves it.
__global__ void __launch_bounds__(CH_THREADS)
    cholesky_diag_kernel(float* __restrict__ a, int64_t lda, int nb, int64_t offset,
                         int32_t* __restrict__ info) {
  __shared__ float col[2][CH_NB];
  const int t = threadIdx.x;
  const int bi = t / CH_GRID, bj = t % CH_GRID;
  const bool active = bj <= bi;
  const int i0 = bi * CH_SB, j0 = bj * CH_SB;

  float v[CH_SB][CH_SB];
#pragma unroll
  for (int r = 0; r < CH_SB; ++r) {
#pragma unroll
    for (int c = 0; c < CH_SB; ++c) {
      const int i = i0 + r, j = j0 + c;
      float x = 0.0f;
      if (i >= nb || j >= nb)
        x = (i == j) ? 1.0f : 0.0f;
      else if (active && j <= i)
        x = a[(int64_t)i * lda + j];
      v[r][c] = x;
    }
  }
  if (bj == 0) {
#pragma unroll
    for (int r = 0; r < CH_SB; ++r) col[0][i0 + r] = v[r][0];
  }
  __syncthreads();

  // Only lower-triangle elements are ever published or stored, so the
  // updates below run unmasked over whole sub-blocks: what they write above
  // the diagonal (from stale column entries of rows < k) is never read.
  bool failed = false;
  for (int kb = 0; kb < CH_GRID; ++kb) {
#pragma unroll
    for (int kc = 0; kc < CH_SB; ++kc) {
      const int k = kb * CH_SB + kc;
      const float* ck = col[kc & 1];
      const float d = ck[k];
      if (t == 0 && !failed && !(d > 0.0f)) {
        failed = true;
        atomicCAS(info, 0, (int32_t)(offset + k + 1));
      }
      const float s = sqrtf(d);
      const float rs = 1.0f / s;
      if (active && bj >= kb) {
        float li[CH_SB], lj[CH_SB];
#pragma unroll
        for (int r = 0; r < CH_SB; ++r) li[r] = ck[i0 + r] * rs;
#pragma unroll
        for (int c = 0; c < CH_SB; ++c) lj[c] = ck[j0 + c] * rs;
        if (bj == kb) {
          // Column k is final (L[k][k] = s, below it the column times 1/s,
          // the scaling of LAPACK's potf2); columns after it are updated.
#pragma unroll
          for (int r = 0; r < CH_SB; ++r) v[r][kc] = li[r];
          if (bi == kb) v[kc][kc] = s;
#pragma unroll
          for (int r = 0; r < CH_SB; ++r) {
#pragma unroll
            for (int c = kc + 1; c < CH_SB; ++c) v[r][c] = fmaf(-li[r], lj[c], v[r][c]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < CH_SB; ++r) {
#pragma unroll
            for (int c = 0; c < CH_SB; ++c) v[r][c] = fmaf(-li[r], lj[c], v[r][c]);
          }
        }
        // Publish column k + 1 for the next step.
        const int nkb = (kc == CH_SB - 1) ? kb + 1 : kb;
        if (bj == nkb) {
#pragma unroll
          for (int r = 0; r < CH_SB; ++r) col[(kc + 1) & 1][i0 + r] = v[r][(kc + 1) % CH_SB];
        }
      }
      __syncthreads();
    }
  }
  // L on and below the diagonal, zeros above.
#pragma unroll
  for (int r = 0; r < CH_SB; ++r) {
#pragma unroll
    for (int c = 0; c < CH_SB; ++c) {
      const int i = i0 + r, j = j0 + c;
      if (i < nb && j < nb) a[(int64_t)i * lda + j] = (j <= i && active) ? v[r][c] : 0.0f;
    }
  }
}

// ------------------------------------------------------------ LDLQ steps

// Index of the block holding batch tile `tile` (blocks sorted by tile0).
__device__ __forceinline__ int ldlq_block_of(const exl3_ldlq_block* __restrict__ blocks,
                                             int nblocks, int64_t tile) {
  int b = 0;
  while (b + 1 < nblocks && blocks[b + 1].tile0 <= tile) ++b;
  return b;
}

__global__ void __launch_bounds__(256)
    ldlq_gather_kernel(const exl3_ldlq_block* __restrict__ blocks, int nblocks,
                       float* __restrict__ x) {
  const int64_t tile = blockIdx.x;
  const exl3_ldlq_block blk = blocks[ldlq_block_of(blocks, nblocks, tile)];
  const int64_t t = tile - blk.tile0;
  // A table that does not cover this tile writes nothing (the host checks
  // the table before it is uploaded).
  if (t < 0 || t >= blk.n / 16) return;
  const int p = threadIdx.x;
  const int e = exl3::tc_perm(p);
  const int64_t off = (int64_t)(e >> 4) * blk.n + t * 16 + (e & 15);
  const float* w = reinterpret_cast<const float*>(blk.w);
  const float* comp = reinterpret_cast<const float*>(blk.comp);
  x[tile * 256 + p] = w[off] + comp[off];
}

__global__ void __launch_bounds__(256)
    ldlq_scatter_kernel(const exl3_ldlq_block* __restrict__ blocks, int nblocks,
                        const float* __restrict__ recon, const int16_t* __restrict__ idx) {
  const int64_t tile = blockIdx.x;
  const exl3_ldlq_block blk = blocks[ldlq_block_of(blocks, nblocks, tile)];
  const int64_t t = tile - blk.tile0;
  if (t < 0 || t >= blk.n / 16) return;
  const int p = threadIdx.x;
  const int e = exl3::tc_perm(p);
  const int64_t off = (int64_t)(e >> 4) * blk.n + t * 16 + (e & 15);
  const float v = recon[tile * 256 + p];
  const float w = reinterpret_cast<const float*>(blk.w)[off];
  reinterpret_cast<float*>(blk.wq)[off] = v;
  reinterpret_cast<float*>(blk.err)[off] = w - v;
  reinterpret_cast<int16_t*>(blk.states)[t * 256 + p] = idx[tile * 256 + p];
}

// Checks the shape and launches the Hadamard kernel variant for (side,
// divisor present, sums of squares wanted).
int launch_hadamard(const float* in, float* out, int64_t rows, int64_t cols, int side,
                    const float* div, float* sumsq, void* stream, const char* what) {
  if (!in || !out) return set_error("%s: NULL buffer", what);
  if (rows <= 0 || cols <= 0) return set_error("%s: empty matrix (%lld x %lld)", what,
                                                (long long)rows, (long long)cols);
  if (side != 0 && side != 1) return set_error("%s: side must be 0 or 1, got %d", what, side);
  if (side == 0 && rows % HAD_N)
    return set_error("%s: rows (%lld) must be divisible by 128", what, (long long)rows);
  if (side == 1 && cols % HAD_N)
    return set_error("%s: columns (%lld) must be divisible by 128", what, (long long)cols);
  hipStream_t st = as_stream(stream);
  if (side == 1) {
    const int64_t seg_per_row = cols / HAD_N;
    const int64_t segments = rows * seg_per_row;
    const int64_t want = (segments + HAD_RIGHT_WAVES - 1) / HAD_RIGHT_WAVES;
    // Grid-stride beyond 65536 workgroups (several segments per wave).
    const int64_t blocks = want < 65536 ? want : 65536;
    const dim3 grid((unsigned)blocks), block(64 * HAD_RIGHT_WAVES);
    if (div && sumsq)
      hipLaunchKernelGGL((had128_right_kernel<true, true>), grid, block, 0, st, in, out, segments,
                         seg_per_row, div, sumsq);
    else if (div)
      hipLaunchKernelGGL((had128_right_kernel<true, false>), grid, block, 0, st, in, out,
                         segments, seg_per_row, div, sumsq);
    else if (sumsq)
      hipLaunchKernelGGL((had128_right_kernel<false, true>), grid, block, 0, st, in, out,
                         segments, seg_per_row, div, sumsq);
    else
      hipLaunchKernelGGL((had128_right_kernel<false, false>), grid, block, 0, st, in, out,
                         segments, seg_per_row, div, sumsq);
  } else {
    const int64_t gx = (cols + 255) / 256, gy = rows / HAD_N;
    if (gx > INT32_MAX || gy > 65535) return set_error("%s: matrix too large", what);
    const dim3 grid((unsigned)gx, (unsigned)gy), block(256);
    if (div)
      hipLaunchKernelGGL((had128_left_kernel<true>), grid, block, 0, st, in, out, cols, div);
    else
      hipLaunchKernelGGL((had128_left_kernel<false>), grid, block, 0, st, in, out, cols, div);
  }
  return check_launch(what);
}

}  // namespace

// ------------------------------------------------------------------- C-ABI

extern "C" {

int exl3_hadamard128(const float* in, float* out, int64_t rows, int64_t cols, int side,
                     void* stream) {
  return launch_hadamard(in, out, rows, cols, side, nullptr, nullptr, stream, "hadamard128");
}

int exl3_hadamard128_scaled(const float* in, float* out, int64_t rows, int64_t cols, int side,
                            const float* divisor, float* slice_sumsq, void* stream) {
  if (slice_sumsq && side != 1)
    return set_error("hadamard128_scaled: slice sums of squares need side = 1");
  return launch_hadamard(in, out, rows, cols, side, divisor, slice_sumsq, stream,
                         "hadamard128_scaled");
}

int exl3_block_rms_from_slices(const float* slice_sumsq, float* out, int64_t outputs, int64_t n,
                               int64_t slices, void* stream) {
  if (!slice_sumsq || !out) return set_error("block_rms_from_slices: NULL buffer");
  if (outputs <= 0 || n <= 0 || slices <= 0)
    return set_error("block_rms_from_slices: empty shape (%lld outputs, n %lld, %lld slices)",
                     (long long)outputs, (long long)n, (long long)slices);
  unsigned b;
  if (exl3::grid_1d(outputs, 256, &b, "block_rms_from_slices")) return 1;
  hipLaunchKernelGGL(block_rms_reduce_kernel, dim3(b), dim3(256), 0, as_stream(stream),
                     slice_sumsq, out, outputs, n, slices, 1);
  return check_launch("block_rms_from_slices");
}

int64_t exl3_block_rms_workspace(int64_t rows, int64_t cols, int dim, int blocksize) {
  if (rows <= 0 || cols <= 0 || (dim != 0 && dim != 1) || blocksize <= 0) return -1;
  const int64_t outputs = dim == 0 ? cols : rows, n = dim == 0 ? rows : cols;
  return outputs * ((n + blocksize - 1) / blocksize);
}

int exl3_block_rms(const float* x, float* out, int64_t rows, int64_t cols, int dim, int blocksize,
                   float* workspace, int64_t workspace_elems, void* stream) {
  if (!x || !out || !workspace) return set_error("block_rms: NULL buffer");
  if (rows <= 0 || cols <= 0) return set_error("block_rms: empty matrix");
  if (dim != 0 && dim != 1) return set_error("block_rms: dim must be 0 or 1, got %d", dim);
  if (blocksize <= 0) return set_error("block_rms: blocksize must be positive, got %d", blocksize);
  const int64_t need = exl3_block_rms_workspace(rows, cols, dim, blocksize);
  if (workspace_elems < need)
    return set_error("block_rms: workspace holds %lld floats, %lld needed",
                     (long long)workspace_elems, (long long)need);
  const int64_t outputs = dim == 0 ? cols : rows;
  const int64_t n = dim == 0 ? rows : cols;
  const int64_t so = dim == 0 ? 1 : cols, st = dim == 0 ? cols : 1;
  const int64_t ns = (n + blocksize - 1) / blocksize;
  unsigned b1, b2;
  if (exl3::grid_1d(outputs * ns, 256, &b1, "block_rms")) return 1;
  if (exl3::grid_1d(outputs, 256, &b2, "block_rms")) return 1;
  hipStream_t sm = as_stream(stream);
  hipLaunchKernelGGL(block_rms_slices_kernel, dim3(b1), dim3(256), 0, sm, x, workspace, outputs, n,
                     so, st, blocksize, ns, dim);
  if (check_launch("block_rms")) return 1;
  hipLaunchKernelGGL(block_rms_reduce_kernel, dim3(b2), dim3(256), 0, sm, workspace, out, outputs,
                     n, ns, dim);
  return check_launch("block_rms");
}

int exl3_cholesky_diag_block(float* a, int64_t lda, int nb, int64_t offset, int32_t* info,
                             void* stream) {
  if (!a || !info) return set_error("cholesky_diag_block: NULL buffer");
  if (nb < 1 || nb > CH_NB)
    return set_error("cholesky_diag_block: block order must be in 1..%d, got %d", CH_NB, nb);
  if (lda < nb) return set_error("cholesky_diag_block: lda (%lld) < block order (%d)",
                                 (long long)lda, nb);
  if (offset < 0) return set_error("cholesky_diag_block: negative offset");
  hipLaunchKernelGGL(cholesky_diag_kernel, dim3(1), dim3(CH_THREADS), 0, as_stream(stream), a, lda,
                     nb, offset, info);
  return check_launch("cholesky_diag_block");
}

int exl3_cholesky_block_order(void) { return CH_NB; }

int exl3_ldlq_gather(const exl3_ldlq_block* blocks, int nblocks, int64_t tiles, float* x,
                     void* stream) {
  if (!blocks || !x) return set_error("ldlq_gather: NULL buffer");
  if (nblocks < 1) return set_error("ldlq_gather: no blocks");
  if (tiles < 1 || tiles > INT32_MAX) return set_error("ldlq_gather: bad tile count %lld",
                                                       (long long)tiles);
  hipLaunchKernelGGL(ldlq_gather_kernel, dim3((unsigned)tiles), dim3(256), 0, as_stream(stream),
                     blocks, nblocks, x);
  return check_launch("ldlq_gather");
}

int exl3_ldlq_scatter(const exl3_ldlq_block* blocks, int nblocks, int64_t tiles,
                      const float* recon, const int16_t* idx, void* stream) {
  if (!blocks || !recon || !idx) return set_error("ldlq_scatter: NULL buffer");
  if (nblocks < 1) return set_error("ldlq_scatter: no blocks");
  if (tiles < 1 || tiles > INT32_MAX) return set_error("ldlq_scatter: bad tile count %lld",
                                                       (long long)tiles);
  hipLaunchKernelGGL(ldlq_scatter_kernel, dim3((unsigned)tiles), dim3(256), 0, as_stream(stream),
                     blocks, nblocks, recon, idx);
  return check_launch("ldlq_scatter");
}

}  // extern "C"
