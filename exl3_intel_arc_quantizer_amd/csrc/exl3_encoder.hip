// MI355X (gfx950) EXL3 trellis tile encoder: HIP kernels + C-ABI.
//
// Path: the two-pass tail-biting Viterbi search of the reference's
// ReferenceTrellisEncoder.encode_tile (exl3_quant/reference_encoder.py:253-324)
// and its SYCL kernel FusedQuantizeKernel (quantize_kernels.sycl:245-360),
// re-designed for CDNA4:
//
//   acs_forward_rows   K = 1..3, acs_forward_chunked K = 4..8. One
//                      1024-thread workgroup per tile, fp16 path costs
//                      ping-pong in LDS (edge order, or chunk-major so that
//                      a thread's predecessor costs are 16-byte loads), each
//                      thread owns 64 (edge, branch) candidates whose
//                      codebook values stay in 32 VGPRs. A step is a packed
//                      subtract and FMA per candidate pair plus
//                      v_pk_minimum3_f16 folding two pairs per instruction:
//                      the minimum cost per edge only. Every
//                      row_stride(K)-th cost row goes to HBM (group-major,
//                      coalesced stores after the step's arithmetic); the
//                      traceback recomputes the argmin of the one edge on
//                      the path.
//   acs_forward_generic reference-structured kernel (one edge per thread
//                      iteration, codebook decoded per candidate, strict fp16
//                      '<' scan): the force_global_costs variant; writes the
//                      same scratch layout as the fast kernels.
//   traceback_rows_kernel one 64-lane workgroup per tile walks the ring
//                      backwards; one evaluation of each stored row's tree
//                      (rebuilding the costs of the unstored steps) yields
//                      the branches of every step that reads that row.
//   traceback_stream_kernel the same walk for small batches, with every
//                      stored row prefetched whole into an LDS ring by
//                      loader waves.
//   finalize_kernel    packing, path cost, distortion, un-permutation;
//   unpack_kernel      the inverse of the packing (stored-tensor read-back).
//
// Numerics (bit-exact vs the reference on finite / infinite inputs):
//   dh = fp16(val - w) (v_pk_add_f16), err = fma_f16(dh, dh, cost_prev)
//   (v_pk_fma_f16, one rounding, fp16 denormals preserved). Step 0 is the
//   same FMA against an initial cost vector of +0 (unconstrained) or
//   {+0 at pre_state, +inf elsewhere}: fma(dh, dh, +0) == fp16(dh*dh) and
//   fma(dh, dh, +inf) == +inf, which is the reference's masked step 0
//   (reference_encoder.py:152-179).
//   Costs are non-negative fp16 or +inf, whose bit patterns order like their
//   values, so an unsigned min gives the minimum cost, and a min over
//   (cost_bits << 16 | k) picks the lowest k among equal minima — the
//   reference's "k = 0 initialises, later k replaces only if strictly
//   smaller" rule (reference_encoder.py:169-176,193-199). NaN inputs are
//   counted by prepare_kernel and rejected by the host wrapper.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

#include "../../include/exl3_encoder.h"
#include "exl3_errors.h"
#include "exl3_layout.h"

using exl3::RowLayout;

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

#define EXL3_VERSION "exl3-mi355x 0.1.0"

// ------------------------------------------------------------------ errors

using exl3::check_launch;
using exl3::g_last_error;
using exl3::grid_1d;
using exl3::set_error;

// --------------------------------------------------------------- codebook

__device__ __forceinline__ f16 f16_bits(uint32_t b) {
  return __builtin_bit_cast(f16, (uint16_t)b);
}
__device__ __forceinline__ uint16_t bits_f16(f16 h) { return __builtin_bit_cast(uint16_t, h); }

// The codebooks (reference trellis_format.py:41-81, quantize_kernels.sycl:51-73;
// upstream codebook.cuh:56-123) hash state s to x = s * M (+ A for 3INST)
// modulo 2^32 and decode x. The hash is affine in s, so for s = s1 + s2
// (disjoint bit fields) x = hash(s1) + s2 * M: the traceback trees compute
// one product per lane and add compile-time offsets for the other fields,
// instead of a quarter-rate v_mul_lo_u32 per leaf.
__host__ __device__ constexpr uint32_t hash_mult(int cb) {
  return cb == 2 ? 0x83DCD12Du : (cb == 0 ? 89226354u : 0xCBAC1FEDu);
}
__device__ __forceinline__ uint32_t hash_state(int cb, uint32_t s) {
  return s * hash_mult(cb) + (cb == 0 ? 64248484u : 0u);
}
__device__ __forceinline__ f16 decode_hash(int cb, uint32_t x) {
  if (cb == 2) {
    // v_sad_u8(x, 0, 0x6400) = 0x6400 + the sum of x's four bytes (each
    // |byte - 0|) in one instruction; 0x6400 + bsum is the fp16 encoding of
    // 1024 + bsum (bsum <= 1020). One fused fp16 FMA.
    const uint32_t h = __builtin_amdgcn_sad_u8(x, 0u, 0x6400u);
    return __builtin_fmaf16(f16_bits(h), f16_bits(0x1EEEu), f16_bits(0xC931u));
  }
  x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
  return f16_bits(x & 0xFFFFu) + f16_bits(x >> 16);
}

// fp16 value of state s.
__device__ __forceinline__ f16 decode_state(int cb, uint32_t s) {
  return decode_hash(cb, hash_state(cb, s));
}

__global__ void decode_codebook_kernel(int cb, uint16_t* __restrict__ out) {
  const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s < 65536u) out[s] = bits_f16(decode_state(cb, s));
}

// ------------------------------------------------------- tile permutation

using exl3::tc_perm;
using exl3::tc_perm_inv;

// ------------------------------------------------------- shared helpers

__device__ __forceinline__ uint32_t umin(uint32_t a, uint32_t b) { return a < b ? a : b; }

__device__ __forceinline__ uint32_t wave_min(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = umin(v, (uint32_t)__shfl_xor((int)v, m, 64));
  return v;
}

// Edge-to-LDS-position maps, passed to the shared prologue, epilogue and
// argmin helpers: EdgePos keeps the cost vector in edge order (the generic
// kernel and K = 1..3); ChunkMap<K> below is the chunk-major layout of
// K = 4..8.
struct EdgePos {
  __device__ static __forceinline__ int at(int x) { return x; }
};

// Lowest-index minimum of the terminal costs (reference argmin_cost,
// reference_encoder.py:206-214): key = cost_bits << 16 | edge; all +inf
// gives edge 0. Result broadcast to all threads via s_red[0].
template <int NT, class Pos = EdgePos>
__device__ uint32_t block_argmin(const uint16_t* cost, int E, uint32_t* s_red) {
  uint32_t best = 0xFFFFFFFFu;
  for (int e = threadIdx.x; e < E; e += NT)
    best = umin(best, ((uint32_t)cost[Pos::at(e)] << 16) | (uint32_t)e);
  best = wave_min(best);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t b = s_red[0];
    for (int w = 1; w < NT / 64; ++w) b = umin(b, s_red[w]);
    s_red[0] = b;
  }
  __syncthreads();
  return s_red[0] & 0xFFFFu;
}

// Arguments shared by the forward kernels. Tile t of the launch reads
// in + t*L and owns scratch block t.
struct FwdArgs {
  const float* in;
  int n, L, roll, cb;
  int store_from;             // step rows i in [store_from, L-2] are stored
  const int32_t* pre_states;  // may be NULL: unconstrained
  int64_t pre_stride;         // in int32 elements
  uint8_t* scratch;           // per-tile blocks of (L+1) rows
  int64_t tile_stride;        // bytes per block
  int64_t hdr_offset;         // byte offset of the header row inside a block
  uint16_t* term_costs;       // [tile][2][E] or NULL
  int cost_slot;
  int32_t* best_edges;        // terminal argmin per tile or NULL
  int64_t best_stride;
};

// Load the tile's fp16 inputs into LDS, record pre_state (and, for cost rows,
// the inputs) in the tile header, and set the initial cost vector. s_w is in
// ring order (s_w[ri]), or with step_order in step order (s_w[i] = input
// (i + roll) mod L).
template <int NT, class Pos = EdgePos>
__device__ __forceinline__ void forward_prologue(const FwdArgs& a, int E, bool stash_inputs,
                                                 f16* s_w, uint16_t* cost0, int& pre_out,
                                                 bool step_order = false) {
  const int tile = blockIdx.x;
  const float* in = a.in + (int64_t)tile * a.L;
  uint8_t* hdr = a.scratch + (int64_t)tile * a.tile_stride + a.hdr_offset;
  for (int r = threadIdx.x; r < a.L; r += NT) {
    const f16 w = (f16)in[r];
    int slot = r;
    if (step_order) {
      slot = r - a.roll;
      if (slot < 0) slot += a.L;
    }
    s_w[slot] = w;
    if (stash_inputs) reinterpret_cast<uint16_t*>(hdr + exl3::HDR_W_BYTES)[r] = bits_f16(w);
  }
  const int pre = a.pre_states ? a.pre_states[(int64_t)tile * a.pre_stride] : -1;
  if (threadIdx.x == 0) reinterpret_cast<int32_t*>(hdr)[exl3::HDR_PRE_STATE] = pre;
  for (int e = threadIdx.x; e < E; e += NT)
    cost0[Pos::at(e)] = (pre < 0 || e == pre) ? 0 : 0x7C00;
  pre_out = pre;
}

// Terminal costs to temp_costs and the pass-1 terminal argmin.
template <int NT, class Pos = EdgePos>
__device__ __forceinline__ void forward_epilogue(const FwdArgs& a, int E, const uint16_t* cfin,
                                                 uint32_t* s_red) {
  const int tile = blockIdx.x;
  if (a.term_costs) {
    uint16_t* dst = a.term_costs + ((int64_t)tile * 2 + a.cost_slot) * E;
    for (int e = threadIdx.x; e < E; e += NT) dst[e] = cfin[Pos::at(e)];
  }
  if (a.best_edges) {
    const uint32_t b = block_argmin<NT, Pos>(cfin, E, s_red);
    if (threadIdx.x == 0) a.best_edges[(int64_t)tile * a.best_stride] = (int32_t)b;
  }
}

// Copy the cost row of step `step` (held in LDS in edge order) to its slot
// in the tile's scratch: position t holds edge exl3::cost_row_edge(K, t)
// (group-major, (h << K) | k for edge (k << (16-2K)) | h). 16-byte chunk c covers
// positions 8c .. 8c + 7, gathered from LDS; the global stores stay
// contiguous. The chunks go to the first E / 8 threads: leaving the other
// waves free measured faster than spreading the gather over every wave.
template <int NT>
__device__ __forceinline__ void store_cost_row(const FwdArgs& a, int K, const uint16_t* src,
                                               int step) {
  const RowLayout lay = exl3::make_layout(K);
  const int E = 65536 >> K;
  const int chunks = E / 8;
  uint4* dst = reinterpret_cast<uint4*>(a.scratch + (int64_t)blockIdx.x * a.tile_stride +
                                        (int64_t)exl3::cost_row_slot(lay, step) * lay.row_bytes);
  for (int c = threadIdx.x; c < chunks; c += NT) {
    uint32_t v[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int t0 = 8 * c + 2 * m, t1 = t0 + 1;
      const uint32_t lo = src[exl3::cost_row_edge(K, t0)];
      const uint32_t hi = src[exl3::cost_row_edge(K, t1)];
      v[m] = lo | (hi << 16);
    }
    dst[c] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// store_cost_row for the edge-order kernel (K = 1..3), run after a step's
// arithmetic (the stored row, the step's input, stays intact until the
// barrier): 16-byte pieces of 8 consecutive positions, the first threads
// taking one or more each; a wave's global store stays contiguous. Each
// step writes up to 8 KiB of rows here (2.7 TB/s at 4096 tiles): streaming
// stores measured 80-83 -> 88 % (K = 2) and 87 -> 92-94 % (K = 3) of the
// VALU peak.
template <int K, int NT>
struct RowGather {
  static_assert(K >= 1 && K <= 3, "K = 4..8 gather from the chunk-major layout");
  static constexpr int E = 65536 >> K;
  static constexpr int PIECES = E / 8;
  static constexpr int PPT = (PIECES + NT - 1) / NT;  // pieces per thread
  typedef uint32_t vec __attribute__((ext_vector_type(4)));

  __device__ __forceinline__ static void store(const FwdArgs& a, const uint16_t* src, int step) {
    constexpr int ks = 16 - 2 * K;
    const RowLayout lay = exl3::make_layout(K);
    vec* dst = reinterpret_cast<vec*>(a.scratch + (int64_t)blockIdx.x * a.tile_stride +
                                      (int64_t)exl3::cost_row_slot(lay, step) * lay.row_bytes);
    if constexpr (K > 1) {
      static_assert(exl3::cost_row_tree_bits(K) > 0, "K = 2, 3 rows are tree-major");
      // Positions t and t + E/2 hold the LDS neighbours x and x + 1 (x
      // even): the first E/16 threads take pieces c and c + E/16 each, from
      // eight dword reads, their halves sorted into the two pieces by
      // v_perm. A dword's LDS bank is edge bits x1 .. x6, so each half-wave
      // takes the 32 pieces that differ in x1 .. x5 (32 different banks per
      // read), and a wave's 64 pieces are 8 runs of 8: 8 whole 128-byte
      // lines per store.
      constexpr int HALF = PIECES / 2;
      static_assert(HALF <= NT && HALF % 64 == 0, "one pair of pieces per thread");
      const int tid = threadIdx.x;
      const int lane = tid & 63, w = tid >> 6;
      int c;
      if constexpr (K == 2) {
        // Piece bits 0..9 are positions 3..12 = edge bits x11, x4 .. x9, x1,
        // x2, x3: a half-wave spans x1 .. x5, its halves differ in x11, the
        // 16 waves in x6 .. x9.
        c = ((lane >> 5) & 1) | ((lane & 24) >> 2) | ((lane & 7) << 7) | ((w & 15) << 3);
      } else {
        // Piece bits 0..8 are positions 3..11 = edge bits x4 .. x9, x1, x2,
        // x3: a half-wave spans x1 .. x5, its halves differ in x6, the 8
        // gathering waves in x7 .. x9.
        c = (lane & 3) | ((lane & 28) << 4) | (((lane >> 5) & 1) << 2) | ((w & 7) << 3);
      }
      if (HALF == NT || tid < HALF) {
        const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
        uint32_t r[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) r[u] = s32[exl3::cost_row_edge(K, 8 * c + u) >> 1];
        vec lo, hi;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          lo[m] = __builtin_amdgcn_perm(r[2 * m + 1], r[2 * m], 0x05040100u);
          hi[m] = __builtin_amdgcn_perm(r[2 * m + 1], r[2 * m], 0x07060302u);
        }
        __builtin_nontemporal_store(lo, &dst[c]);
        __builtin_nontemporal_store(hi, &dst[c + HALF]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < PPT; ++j) {
        const int c = threadIdx.x + j * NT;
        if (PIECES % NT == 0 || c < PIECES) {
          // Even positions 8c + 2m from block 0, odd ones from block 1, each
          // four LDS neighbours (4c .. 4c + 3): two 8-byte reads.
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 e = *reinterpret_cast<const u32x2*>(src + 4 * c);
          const u32x2 o = *reinterpret_cast<const u32x2*>(src + (1 << ks) + 4 * c);
          vec v;
          v[0] = __builtin_amdgcn_perm(o.x, e.x, 0x05040100u);
          v[1] = __builtin_amdgcn_perm(o.x, e.x, 0x07060302u);
          v[2] = __builtin_amdgcn_perm(o.y, e.y, 0x05040100u);
          v[3] = __builtin_amdgcn_perm(o.y, e.y, 0x07060302u);
          __builtin_nontemporal_store(v, &dst[c]);
        }
      }
    }
  }
};

// Whether forward step i stores the cost row of step i - 1.
__device__ __forceinline__ bool stores_row(const FwdArgs& a, int K, int i) {
  return i >= 1 && i - 1 >= a.store_from && exl3::cost_row_stored(exl3::make_layout(K), i - 1);
}

// stores_row for a step of known parity (i = 2 p + B): rows are stored at
// steps i - 1 that are multiples of an even stride, so an even step never
// stores one unless the stride is 1.
template <int K, int B>
__device__ __forceinline__ bool stores_row_at(const FwdArgs& a, int i) {
  constexpr int STRIDE = exl3::row_stride(K);
  if constexpr (STRIDE > 1 && STRIDE % 2 == 0 && B == 0) {
    return false;
  } else {
    return i - 1 >= a.store_from &&
           (STRIDE == 1 || (STRIDE == 2 && B == 1) || (i - 1) % STRIDE == 0);
  }
}

template <int V>
struct Phase {
  static constexpr int value = V;
};

// ------------------------------------------------------------ fast kernels

// Thread decomposition of the edge-order kernel (K = 1..3): G groups x J
// edges x 2^K branches per thread; 1024 threads, 64 candidates per thread
// and step.
template <int K>
struct FastShape {
  static_assert(K >= 1 && K <= 3, "K = 4..8 use the chunk-major kernel");
  static constexpr int G = (K == 1) ? 16 : (K == 2 ? 4 : 1);
  static constexpr int J = (K == 1) ? 2 : (K == 2 ? 4 : 8);
};

template <int K, int G, int J>
struct FastCfg {
  static constexpr int E = 65536 >> K;
  static constexpr int S = 65536 >> (2 * K);  // groups
  static constexpr int Q = 1 << K;            // branches
  static constexpr int NJ = Q / J;            // edge sets per group set
  static constexpr int NGQ = S / G;           // group sets
  static constexpr int NT = NGQ * NJ;         // threads per tile
  static constexpr int KR = 16 - K;
  static_assert(NT == 1024, "fast configurations use 1024 threads");
  static_assert(J % 2 == 0, "edges are processed in packed pairs (j, j + 1)");
  static_assert(G == 1 || G % 2 == 0, "groups are read in 32-bit pairs");
};

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Minimum over the P neighbouring lanes that split one output pair's
// branches (P = 1, 2, 4, 8), left in every one of them.
template <int P>
__device__ __forceinline__ u16x2 group_min_u16x2(u16x2 v) {
  if (P >= 2) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(
        0, (int)__builtin_bit_cast(uint32_t, v), 0xB1, 0xF, 0xF, false);
    v = __builtin_elementwise_min(v, __builtin_bit_cast(u16x2, o));
  }
  if (P >= 4) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(
        0, (int)__builtin_bit_cast(uint32_t, v), 0x4E, 0xF, 0xF, false);
    v = __builtin_elementwise_min(v, __builtin_bit_cast(u16x2, o));
  }
  if (P >= 8) {
    // Each quad now holds its minimum; row_half_mirror pairs lane i with
    // lane 7 - i of its half row, which lies in the other quad.
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(
        0, (int)__builtin_bit_cast(uint32_t, v), 0x141, 0xF, 0xF, false);
    v = __builtin_elementwise_min(v, __builtin_bit_cast(u16x2, o));
  }
  return v;
}

// Edge-order forward pass (K = 1..3): minimum cost per edge, rows to HBM.
// Thread `unit` owns edges jj*J .. jj*J + J - 1 of G groups (one group, or
// NV runs of GV consecutive groups when G > 1), in packed pairs (j, j + 1),
// and all 2^K branches k. All edges of a group share the 2^K predecessor
// costs, so each cost is broadcast to both halves of the FMA addend
// (op_sel) from a 16-bit LDS read (G = 1) or one half of a 32-bit read
// holding two groups' costs (G > 1). v_pk_minimum3_f16 folds two candidates
// per instruction into the running minimum (costs are non-negative fp16
// with no NaN, where IEEE minimum returns the same bits as an integer
// minimum). The pair minima are in edge order for 32-bit LDS stores. CB is
// the codebook selector (compile time keeps the prologue's registers low).
// Eight waves per SIMD: two workgroups per CU, which caps VGPRs at 64.
// K = 1's ping-pong pair of cost vectors takes 128 KiB of LDS, one
// workgroup per CU; INPLACE keeps one vector (64 KiB) and updates it in
// place, with a second barrier per step between the reads and the writes:
// two workgroups per CU, 10 % faster at 1024 tiles and more, 3 % slower
// where one workgroup per CU is all the batch fills.
template <int K, int G, int J, int CB, bool INPLACE>
__global__ void __launch_bounds__(1024, (K == 1 && !INPLACE ? 4 : 8)) acs_forward_rows(FwdArgs a) {
  using C = FastCfg<K, G, J>;
  constexpr int JP = J / 2;
  static_assert(C::Q % 2 == 0, "branches are folded two at a time");
  static_assert(!INPLACE || K == 1, "the in-place update is written for K = 1");
  __shared__ __attribute__((aligned(16))) uint16_t s_cost[INPLACE ? 1 : 2][C::E];
  __shared__ __attribute__((aligned(4))) f16 s_w[256];
  __shared__ uint32_t s_red[16];

  const int L = a.L;
  const int tid = threadIdx.x;
  const int unit = tid;
  const int jj = unit % C::NJ;
  // G > 1 (K = 1, 2): the thread's groups form NV runs of GV consecutive
  // groups, one 16-byte vector of pair minima each, SV groups apart; lanes
  // own adjacent runs, so each output vector store is contiguous over the
  // wave (bank-conflict free) and each predecessor read is too.
  constexpr int GV = G > 1 ? (8 >> K) : 1;
  constexpr int NV = G / GV;
  constexpr int SV = C::S / NV;
  static_assert(G % GV == 0 && (G == 1 || GV % 2 == 0), "runs hold whole group pairs");
  const int hbase = (unit / C::NJ) * GV;
  auto grp = [&](int g) { return (g / GV) * SV + hbase + (g % GV); };

  f16x2 cbv[G][JP][C::Q];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int jp = 0; jp < JP; ++jp)
#pragma unroll
      for (int q = 0; q < C::Q; ++q) {
        const uint32_t s_lo = ((uint32_t)q << C::KR) | ((uint32_t)grp(g) << K) |
                              (uint32_t)(jj * J + 2 * jp);
        f16x2 v;
        v.x = decode_state(CB, s_lo);
        v.y = decode_state(CB, s_lo + 1u);
        cbv[g][jp][q] = v;
      }
  int pre;
  forward_prologue<C::NT>(a, C::E, true, s_w, s_cost[0], pre, true);
  __syncthreads();

  // One step; B = i & 1 is the ping-pong phase, fixed at compile time so
  // every LDS address is a per-thread base plus an immediate offset.
  auto step = [&](auto phase, int i, f16 w) {
    constexpr int B = decltype(phase)::value;
    const uint16_t* cin = s_cost[INPLACE ? 0 : B];
    uint32_t* cout = reinterpret_cast<uint32_t*>(s_cost[INPLACE ? 0 : B ^ 1]);
    const bool store = i >= 1 && stores_row_at<K, B>(a, i);
    f16x2 w2;
    w2.x = w;
    w2.y = w;
    if constexpr (INPLACE) {
      static_assert(C::Q == 2 && JP == 1 && G % 2 == 0, "K = 1 shape");
      // Both predecessor costs (k = 0, 1) of every group are read, and the
      // stored row gathered, before the barrier; the new costs after it.
      uint32_t cw[2][G / 2];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int g2 = 0; g2 < G / 2; ++g2)
          cw[b][g2] = *reinterpret_cast<const uint32_t*>(cin + b * C::S + grp(2 * g2));
      if (store) RowGather<K, C::NT>::store(a, cin, i - 1);
      __syncthreads();
#pragma unroll
      for (int g = 0; g < G; ++g) {
        f16x2 cv[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const f16x2 pair = __builtin_bit_cast(f16x2, cw[b][g >> 1]);
          cv[b] = (g & 1) ? __builtin_shufflevector(pair, pair, 1, 1)
                          : __builtin_shufflevector(pair, pair, 0, 0);
        }
        const f16x2 d0 = cbv[g][0][0] - w2;
        const f16x2 d1 = cbv[g][0][1] - w2;
        const f16x2 e0 = __builtin_elementwise_fma(d0, d0, cv[0]);
        const f16x2 e1 = __builtin_elementwise_fma(d1, d1, cv[1]);
        const int e = (grp(g) << K) | (jj * J);
        cout[e >> 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_minimum(e0, e1));
      }
      __syncthreads();
      return;
    }

    f16x2 m[G][JP];
#pragma unroll
    for (int k = 0; k < C::Q; k += 2) {
      // cw[b][g2]: predecessor costs of branch k (b = 0) and k + 1 (b = 1)
      // for groups grp(2 g2) (low half) and grp(2 g2) + 1 (high half).
      uint32_t cw[2][(G + 1) / 2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const uint16_t* src = cin + (k + b) * C::S;
        if constexpr (G == 1) {
          cw[b][0] = src[grp(0)];
        } else {
#pragma unroll
          for (int g2 = 0; g2 < G / 2; ++g2)
            cw[b][g2] = *reinterpret_cast<const uint32_t*>(src + grp(2 * g2));
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        f16x2 cv[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const f16x2 pair = __builtin_bit_cast(f16x2, cw[b][g >> 1]);
          cv[b] = (g & 1) ? __builtin_shufflevector(pair, pair, 1, 1)
                          : __builtin_shufflevector(pair, pair, 0, 0);
        }
#pragma unroll
        for (int jp = 0; jp < JP; ++jp) {
          const f16x2 d0 = cbv[g][jp][k] - w2;
          const f16x2 d1 = cbv[g][jp][k + 1] - w2;
          const f16x2 e0 = __builtin_elementwise_fma(d0, d0, cv[0]);
          const f16x2 e1 = __builtin_elementwise_fma(d1, d1, cv[1]);
          m[g][jp] = (k == 0) ? __builtin_elementwise_minimum(e0, e1)
                              : __builtin_elementwise_minimum(
                                    __builtin_elementwise_minimum(m[g][jp], e0), e1);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int jp = 0; jp < JP; ++jp) {
        const int e = (grp(g) << K) | (jj * J + 2 * jp);
        cout[e >> 1] = __builtin_bit_cast(uint32_t, m[g][jp]);
      }
    if (store) RowGather<K, C::NT>::store(a, cin, i - 1);
    __syncthreads();
  };
  // L is even: steps go in pairs, whose inputs are one aligned 32-bit read.
  for (int i = 0; i < L; i += 2) {
    const f16x2 wp = *reinterpret_cast<const f16x2*>(&s_w[i]);
    step(Phase<0>(), i, wp.x);
    step(Phase<1>(), i + 1, wp.y);
  }
  forward_epilogue<C::NT>(a, C::E, s_cost[0], s_red);
}

// ------------------------------------------------ chunk-major kernels (K >= 4)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Chunk-major LDS layouts of the cost vector for K = 4..8. Edge x = (k << KS)
// | h (KS = 16 - 2K; k the branch digit a group's threads compare, h the
// group) sits at 8 * phys((h << (K - 3)) | (k >> 3)) + (k & 7): a group's 2^K
// predecessor costs are 2^(K-3) chunks of 16 bytes, each one LDS load. phys
// permutes the chunk slots by XOR-ing low slot bits with higher ones (its
// own inverse), chosen per K so that the loads, the output stores and the
// row gather of every wave spread over the banks.
//
// ChunkMap<K>(tid) is thread tid's share of a step: group h, lane p of the
// P lanes that split its 2^K branches (Q = 2^K / P each, NCH = Q / 8
// chunks), and J outputs x(j) (edges (h << K) | x(j), packed in pairs
// (2 jp, 2 jp + 1)). rd(c) is the LDS element offset of its c-th chunk load
// and kof(c, m) the branch of element m of that chunk; wr(j) is the offset
// of output j (DWORD_OUT: of the pair (x(0), x(1)), adjacent in LDS, stored
// as one dword by lane p = 0). W is the gather's piece size in positions.
template <int K>
struct ChunkMap;

template <>
struct ChunkMap<4> {
  // Wave w takes the 16 groups h = (gh << 4) | w, gh = lane / 4, so each
  // load instruction reads 16 chunks in 16 different places of the bank
  // row; lane jj = lane % 4 takes x = jj + 4 (j ^ (w >> 3)), whose stores
  // are 128 bytes apart (immediate offsets) and fill eight whole chunks in
  // distinct banks per instruction.
  static constexpr int J = 4, P = 1, NCH = 2, W = 8;
  static constexpr bool DWORD_OUT = false;
  __device__ static __forceinline__ int phys(int s) { return s ^ ((s >> 5) & 15); }
  __device__ static __forceinline__ int at(int x) {
    return phys(((x & 255) << 1) | (x >> 11)) * 8 + ((x >> 8) & 7);
  }
  int h, p, jj, xs, r0, r1, wb;
  __device__ explicit ChunkMap(int tid) {
    const int w = tid >> 6, lane = tid & 63;
    jj = lane & 3;
    h = ((lane >> 2) << 4) | w;
    p = 0;
    xs = (w >> 3) & 1;
    r0 = phys(h << 1) * 8;
    r1 = phys((h << 1) | 1) * 8;
    wb = at((h << 4) | (jj + 4 * xs));
  }
  __device__ int x(int j) const { return jj + 4 * (j ^ xs); }
  __device__ int rd(int c) const { return c ? r1 : r0; }
  __device__ int kof(int c, int m) const { return 8 * c + m; }
  __device__ int wr(int j) const { return wb + 64 * j; }
};

template <>
struct ChunkMap<5> {
  // Wave w takes four groups (h bits 1, 2 from lane / 16, the others from
  // w), lane jj = lane % 16 the outputs x = jj + 16 j. A group's four
  // chunks are contiguous, in an order that depends on h & 3.
  static constexpr int J = 2, P = 1, NCH = 4, W = 8;
  static constexpr bool DWORD_OUT = false;
  __device__ static __forceinline__ int phys(int s) { return s ^ ((s >> 2) & 15); }
  __device__ static __forceinline__ int at(int x) {
    return phys(((x & 63) << 2) | (x >> 9)) * 8 + ((x >> 6) & 7);
  }
  int h, p, jj, rb, w0, w1;
  __device__ explicit ChunkMap(int tid) {
    const int w = tid >> 6, lane = tid & 63;
    jj = lane & 15;
    h = (w & 1) | ((lane >> 4) << 1) | ((w >> 1) << 3);
    p = 0;
    rb = (phys(h << 2) & ~3) * 8;
    w0 = at((h << 5) | jj);
    w1 = at((h << 5) | (jj + 16));
  }
  __device__ int x(int j) const { return jj + 16 * j; }
  __device__ int rd(int c) const { return rb + 8 * c; }
  __device__ int kof(int c, int m) const { return 8 * (c ^ (h & 3)) + m; }
  __device__ int wr(int j) const { return j ? w1 : w0; }
};

template <>
struct ChunkMap<6> {
  // One group per wave (h = w); lanes 2u, 2u + 1 split unit u's 64 branches
  // (lane p loads chunks 2c + p), and unit u takes the pair x = xa, xa + 16
  // (xa = u % 16 + 32 (u / 16)), adjacent in LDS.
  static constexpr int J = 2, P = 2, NCH = 4, W = 2;
  static constexpr bool DWORD_OUT = true;
  __device__ static __forceinline__ int phys(int s) { return s ^ ((s >> 3) & 15); }
  __device__ static __forceinline__ int at(int x) {
    return phys(((x & 15) << 3) | (x >> 7)) * 8 + ((x >> 4) & 7);
  }
  int h, p, jj, xa, rb, wb;
  __device__ explicit ChunkMap(int tid) {
    const int w = tid >> 6, lane = tid & 63;
    h = w;
    p = lane & 1;
    jj = lane >> 1;
    xa = (jj & 15) | ((jj >> 4) << 5);
    rb = ((phys(h << 3) & ~7) + (p ^ (h & 1))) * 8;
    wb = at((h << 6) | xa);
  }
  __device__ int x(int j) const { return xa + 16 * j; }
  __device__ int rd(int c) const { return rb + 16 * c; }
  __device__ int kof(int c, int m) const { return 8 * (2 * (c ^ ((h >> 1) & 3)) + p) + m; }
  __device__ int wr(int) const { return wb; }
};

template <>
struct ChunkMap<7> {
  // Four waves per group (h = w / 4); lanes 4u .. 4u + 3 split unit u's 128
  // branches (lane p loads chunks 4c + p), and unit u takes the pair
  // x = xa, xa + 4 (xa = u % 4 + 8 (u / 4)), adjacent in LDS.
  static constexpr int J = 2, P = 4, NCH = 4, W = 2;
  static constexpr bool DWORD_OUT = true;
  __device__ static __forceinline__ int phys(int s) { return s ^ ((s >> 4) & 3); }
  __device__ static __forceinline__ int at(int x) {
    return phys(((x & 3) << 4) | (x >> 5)) * 8 + ((x >> 2) & 7);
  }
  int h, p, jj, xa, rb, wb;
  __device__ explicit ChunkMap(int tid) {
    const int w = tid >> 6, lane = tid & 63;
    h = w >> 2;
    p = lane & 3;
    jj = ((w & 3) << 4) | (lane >> 2);
    xa = (jj & 3) | ((jj >> 2) << 3);
    rb = ((h << 4) + (p ^ h)) * 8;
    wb = at((h << 7) | xa);
  }
  __device__ int x(int j) const { return xa + 4 * j; }
  __device__ int rd(int c) const { return rb + 32 * c; }
  __device__ int kof(int c, int m) const { return 8 * (4 * c + p) + m; }
  __device__ int wr(int) const { return wb; }
};

template <>
struct ChunkMap<8> {
  // A single group in edge order; lanes 8u .. 8u + 7 split unit u's 256
  // branches (lane p loads chunks 8c + p: eight neighbouring chunks per
  // instruction), and unit u takes the pair x = 2u, 2u + 1.
  static constexpr int J = 2, P = 8, NCH = 4, W = 2;
  static constexpr bool DWORD_OUT = true;
  __device__ static __forceinline__ int at(int x) { return x; }
  int h, p, jj;
  __device__ explicit ChunkMap(int tid) {
    h = 0;
    p = tid & 7;
    jj = tid >> 3;
  }
  __device__ int x(int j) const { return 2 * jj + j; }
  __device__ int rd(int c) const { return (8 * c + p) * 8; }
  __device__ int kof(int c, int m) const { return 8 * (8 * c + p) + m; }
  __device__ int wr(int) const { return 2 * jj; }
};

// Forward pass over ChunkMap<K> (K = 4..8): the arithmetic of
// acs_forward_rows (a packed subtract and FMA per candidate pair,
// v_pk_minimum3_f16 folding two pairs, 80 VALU instructions per thread and
// step, plus the P-lane minimum at K >= 6), with each thread's predecessor
// costs read as NCH 16-byte LDS loads instead of Q two-byte ones. A stored
// row's W-position pieces (cost_row_pos) are runs of one chunk, so the row
// gather is one LDS load and one global store per piece.
template <int K, int CB>
__global__ void __launch_bounds__(1024, 8) acs_forward_chunked(FwdArgs a) {
  using M = ChunkMap<K>;
  constexpr int E = 65536 >> K, KR = 16 - K;
  constexpr int J = M::J, P = M::P, NCH = M::NCH, Q = 8 * NCH, JP = J / 2;
  static_assert(Q * P == (1 << K), "the P lanes of a unit cover every branch");
  __shared__ __attribute__((aligned(16))) uint16_t s_cost[2][E];
  __shared__ __attribute__((aligned(4))) f16 s_w[256];
  __shared__ uint32_t s_red[16];

  const int L = a.L;
  const int tid = threadIdx.x;
  const M map(tid);

  // cbv[jp][kk]: codebook values of branch kof(kk / 8, kk % 8) for the
  // output pair (x(2 jp), x(2 jp + 1)). The state's three fields are
  // disjoint bits and its hash is affine, so every hash is the group's hash
  // plus the other fields times the multiplier: a few products per thread
  // instead of a quarter-rate v_mul_lo_u32 per value.
  const uint32_t HM = hash_mult(CB);
  const uint32_t hh = hash_state(CB, (uint32_t)map.h << K);
  f16x2 cbv[JP][Q];
#pragma unroll
  for (int jp = 0; jp < JP; ++jp)
#pragma unroll
    for (int kk = 0; kk < Q; ++kk) {
      const uint32_t hk = hh + ((uint32_t)map.kof(kk >> 3, kk & 7) << KR) * HM;
      f16x2 v;
      v.x = decode_hash(CB, hk + (uint32_t)map.x(2 * jp) * HM);
      v.y = decode_hash(CB, hk + (uint32_t)map.x(2 * jp + 1) * HM);
      cbv[jp][kk] = v;
    }
  // Row gather: piece t (positions W t .. W t + W - 1 of the stored row) is
  // LDS positions at(cost_row_edge(K, W t)) onwards.
  constexpr int W = M::W, PIECES = E / W;
  typedef uint32_t piece_t __attribute__((ext_vector_type(W / 2)));
  const int gpos = tid < PIECES ? M::at((int)exl3::cost_row_edge(K, (uint32_t)(W * tid))) : 0;
  int pre;
  forward_prologue<1024, M>(a, E, true, s_w, s_cost[0], pre, true);
  __syncthreads();

  auto step = [&](auto phase, int i, f16 wv) {
    constexpr int B = decltype(phase)::value;
    const uint16_t* cin = s_cost[B];
    uint16_t* cout = s_cost[B ^ 1];
    const bool store = i >= 1 && stores_row_at<K, B>(a, i);
    f16x2 w2;
    w2.x = wv;
    w2.y = wv;
    f16x2 m[JP];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const u32x4 cw = *reinterpret_cast<const u32x4*>(cin + map.rd(c));
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        // The element goes through a named copy: __builtin_bit_cast of an
        // ext_vector element expression compiles to a cast of element 0
        // with this hipcc.
        const uint32_t word = cw[d];
        const f16x2 pair = __builtin_bit_cast(f16x2, word);
        const f16x2 cv0 = __builtin_shufflevector(pair, pair, 0, 0);
        const f16x2 cv1 = __builtin_shufflevector(pair, pair, 1, 1);
        const int kk = 8 * c + 2 * d;
#pragma unroll
        for (int jp = 0; jp < JP; ++jp) {
          const f16x2 d0 = cbv[jp][kk] - w2;
          const f16x2 d1 = cbv[jp][kk + 1] - w2;
          const f16x2 e0 = __builtin_elementwise_fma(d0, d0, cv0);
          const f16x2 e1 = __builtin_elementwise_fma(d1, d1, cv1);
          m[jp] = (kk == 0) ? __builtin_elementwise_minimum(e0, e1)
                            : __builtin_elementwise_minimum(
                                  __builtin_elementwise_minimum(m[jp], e0), e1);
        }
      }
    }
    if constexpr (M::DWORD_OUT) {
      static_assert(JP == 1, "one output pair per unit");
      const u16x2 v = group_min_u16x2<P>(__builtin_bit_cast(u16x2, m[0]));
      if (map.p == 0) *reinterpret_cast<uint32_t*>(cout + map.wr(0)) = __builtin_bit_cast(uint32_t, v);
    } else {
      static_assert(P == 1, "2-byte outputs are written by their only lane");
#pragma unroll
      for (int jp = 0; jp < JP; ++jp) {
        cout[map.wr(2 * jp)] = bits_f16(m[jp].x);
        cout[map.wr(2 * jp + 1)] = bits_f16(m[jp].y);
      }
    }
    if (store && tid < PIECES) {
      const RowLayout lay = exl3::make_layout(K);
      piece_t* dst = reinterpret_cast<piece_t*>(a.scratch + (int64_t)blockIdx.x * a.tile_stride +
                                                (int64_t)exl3::cost_row_slot(lay, i - 1) *
                                                    lay.row_bytes);
      dst[tid] = *reinterpret_cast<const piece_t*>(cin + gpos);
    }
    __syncthreads();
  };
  for (int i = 0; i < L; i += 2) {
    const f16x2 wp = *reinterpret_cast<const f16x2*>(&s_w[i]);
    step(Phase<0>(), i, wp.x);
    step(Phase<1>(), i + 1, wp.y);
  }
  forward_epilogue<1024, M>(a, E, s_cost[0], s_red);
}

// --------------------------------------------------------- generic kernel

constexpr int GEN_NT = 256;

// Reference-structured forward pass for any K (reference_encoder.py:130-204,
// quantize_kernels.sycl:83-157): per edge, scan branches k = 0..2^K-1 with a
// strict fp16 '<'; codebook decoded per candidate. It writes the cost rows
// of the fast kernels' scratch layout.
__global__ void __launch_bounds__(GEN_NT) acs_forward_generic(FwdArgs a, int K) {
  __shared__ __attribute__((aligned(16))) uint16_t s_cost[2][32768];
  __shared__ f16 s_w[256];
  __shared__ uint32_t s_red[GEN_NT / 64];

  const int L = a.L;
  const int E = 65536 >> K, KR = 16 - K, NB = 1 << K;
  int pre;
  forward_prologue<GEN_NT>(a, E, true, s_w, s_cost[0], pre);
  __syncthreads();

  for (int i = 0; i < L; ++i) {
    int ri = i + a.roll;
    if (ri >= L) ri -= L;
    const uint16_t* cin = s_cost[i & 1];
    uint16_t* cout = s_cost[(i & 1) ^ 1];
    if (stores_row(a, K, i)) store_cost_row<GEN_NT>(a, K, cin, i - 1);
    const f16 w = s_w[ri];
    for (int e = threadIdx.x; e < E; e += GEN_NT) {
      f16 best = 0;
      for (int k = 0; k < NB; ++k) {
        const uint32_t sigma = ((uint32_t)k << KR) | (uint32_t)e;
        const f16 dh = decode_state(a.cb, sigma) - w;
        const f16 err = __builtin_fmaf16(dh, dh, f16_bits(cin[sigma >> K]));
        if (k == 0 || err < best) best = err;
      }
      cout[e] = bits_f16(best);
    }
    __syncthreads();
  }
  forward_epilogue<GEN_NT>(a, E, s_cost[L & 1], s_red);
}

// Terminal argmin from stored costs (the split API's backward pass reads
// temp_costs, quantize_kernels.sycl:459-461).
__global__ void __launch_bounds__(256) argmin_costs_kernel(const uint16_t* __restrict__ costs,
                                                           int E, int cost_slot,
                                                           int32_t* __restrict__ out) {
  __shared__ uint32_t s_red[4];
  const uint16_t* c = costs + ((int64_t)blockIdx.x * 2 + cost_slot) * E;
  const uint32_t b = block_argmin<256>(c, E, s_red);
  if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)b;
}

// -------------------------------------------------------------- traceback

struct TbArgs {
  const uint8_t* scratch;
  int64_t tile_stride, hdr_offset;
  RowLayout lay;
  int n, L, roll, write, cb;
  const int32_t* start;  // start edge per tile
  int64_t start_stride;
  int32_t* end_out;      // edge reached at ring row 0 (write = 0)
  int64_t end_stride;
  float* out_w;          // write = 1
  int16_t* out_idx;
};

// Walk back over the ring (reference backward, reference_encoder.py:216-251;
// quantize_kernels.sycl:320-333,345-358). write = 0: stop after ring row 0
// and emit the edge reached (the tail-biting end state). write = 1: emit
// every state and its codebook value.

// One 64-lane wave per tile. At step i with edge e the path's
// predecessor branch is the key minimum over k of
// fma(dh, dh, C_{i-1}[(k << (16-2K)) | (e >> K)]) (lowest k among equal
// costs), dh = fp16(value((k << (16-K)) | e) - w_i). If step i-1 is D > 0
// steps past the last stored row r0, those 2^K costs are rebuilt from row r0
// over D levels: level m holds C_{i-1-m} at the positions
//   x_0 = (k_0 << (16-2K)) | (e >> K),  x_{m+1} = (k_{m+1} << (16-2K)) | (x_m >> K)
// indexed by the base-2^K digits (k_0 .. k_m); the leaves (level D) are read
// from row r0, and each level above is, per entry, the minimum over its 2^K
// children of the forward pass's FMA: exactly the value the forward pass
// computed for that edge.
//
// Leaf n = k_0 .. k_D (k_D least significant) lives in lane n >> RLOG,
// register n & (R - 1), R = 2^RLOG leaves per lane, so the lowest digits are
// reduced inside a lane and a lane's leaves are one aligned vector load.
// Once a level has reduced every register bit, the registers of a lane hold
// copies of one value and the remaining digits reduce across lanes with
// xor_min (DPP / permlane swaps). Trees with fewer than 64 leaves are
// replicated over the wave.

// min(v, v of lane ^ mask) for mask = 1 .. 32 without the LDS crossbar:
// DPP quad_perm (1, 2), quad reversal then row_half_mirror (4: i ^ 3 ^ 7),
// row_ror:8 (8), and gfx950's v_permlane16_swap / v_permlane32_swap (16,
// 32: the swapped pair holds each lane's value and its partner's). mask
// must fold to a constant; every lane of the wave must be active.
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v, int ctrl) {
  switch (ctrl) {
    case 0xB1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    case 0x4E: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    case 0x1B: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x1B, 0xF, 0xF, false);
    case 0x141: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false);
    default: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
  }
}

__device__ __forceinline__ uint32_t xor_min(uint32_t v, int mask) {
  switch (mask) {
    case 1: return umin(v, dpp_mov(v, 0xB1));
    case 2: return umin(v, dpp_mov(v, 0x4E));
    case 4: return umin(v, dpp_mov(dpp_mov(v, 0x1B), 0x141));
    case 8: return umin(v, dpp_mov(v, 0x128));
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return umin(r[0], r[1]);
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return umin(r[0], r[1]);
    }
  }
}

template <int N>
struct U16Vec {
  typedef uint16_t type __attribute__((ext_vector_type(N)));
};

template <int K>
__device__ __forceinline__ uint32_t row_pos(uint32_t x) {
  return exl3::cost_row_pos(K, x);
}

// The states a traceback tree decodes, split into the part that depends on
// the lane (and the walk's edge) and the part that depends on the register
// index r. Leaf n = (lane << RLOG | r) & (2^(K(D+1)) - 1); every bit of the
// state at level m is a copy of one bit of n or of the edge, so the state is
// the disjoint OR (= sum) of its value with r = 0 and its value with lane = 0
// and edge = 0. hash_state is affine, so the hash of the leaf's state is the
// lane's hash (one multiply per level) plus a compile-time offset per r.
template <int K, int D, int RLOG>
struct TreeFields {
  static constexpr int NB = 1 << K, KR = 16 - K, KS = 16 - 2 * K;
  static constexpr int NLOG = K * (D + 1);
  static constexpr uint32_t NMASK = (1u << NLOG) - 1u;
  uint32_t nl, h0;

  __device__ __forceinline__ TreeFields(int lane, uint32_t edge_hi)
      : nl(((uint32_t)lane << RLOG) & NMASK), h0(edge_hi) {}

  // x_m of leaf n (the predecessor edge at level m) with edge part hh.
  __host__ __device__ static constexpr uint32_t x_at(uint32_t n, uint32_t hh, int m) {
    uint32_t x = ((n >> (K * D)) << KS) | hh;
    for (int j = 1; j <= m; ++j) x = (((n >> (K * (D - j))) & (NB - 1)) << KS) | (x >> K);
    return x;
  }
  // State decoded at level m (digit k_{m+1} over x_m).
  __host__ __device__ static constexpr uint32_t level_state(uint32_t n, uint32_t hh, int m) {
    const int lo = K * (D - 1 - m);
    return (((n >> lo) & (NB - 1)) << KR) | x_at(n, hh, m);
  }
  __device__ __forceinline__ uint32_t level_hash(int cb, int m) const {
    return hash_state(cb, level_state(nl, h0, m));
  }
  __host__ __device__ static constexpr uint32_t level_offset(int cb, int m, int r) {
    return level_state((uint32_t)r & NMASK, 0u, m) * hash_mult(cb);
  }
  // State decoded at the top (digit k_0 over the walk's edge).
  __device__ __forceinline__ uint32_t top_hash(int cb, uint32_t edge) const {
    return hash_state(cb, ((nl >> (K * D)) << KR) | edge);
  }
  __host__ __device__ static constexpr uint32_t top_offset(int cb, int r) {
    return ((((uint32_t)r & NMASK) >> (K * D)) << KR) * hash_mult(cb);
  }
};

template <int K, int CB, int D, bool INIT>
__device__ __forceinline__ uint32_t tb_branch(const uint16_t* __restrict__ leaf, uint32_t edge,
                                              const uint16_t* __restrict__ wbits, int ri, int L,
                                              int lane, int pre) {
  constexpr int NB = 1 << K, KS = 16 - 2 * K;
  constexpr int NLOG = K * (D + 1);
  constexpr int RLOG = NLOG > 6 ? NLOG - 6 : 0;
  constexpr int R = 1 << RLOG;
  constexpr uint32_t NMASK = (1u << NLOG) - 1u;
  constexpr int CH = R < NB ? R : NB;  // leaves per contiguous load
  const uint32_t h0 = edge >> K;

  uint32_t nid[R];
  uint32_t xs[R][D + 1];
  uint32_t v[R];
  TreeFields<K, D, RLOG> tf(lane, h0);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t n = (((uint32_t)lane << RLOG) | (uint32_t)r) & NMASK;
    nid[r] = n;
    uint32_t x = ((n >> (K * D)) << KS) | h0;
    xs[r][0] = x;
#pragma unroll
    for (int m = 1; m <= D; ++m) {
      x = (((n >> (K * (D - m))) & (NB - 1)) << KS) | (x >> K);
      xs[r][m] = x;
    }
  }
  if constexpr (INIT) {
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = (pre < 0 || (int)xs[r][0] == pre) ? 0u : 0x7C00u;
  } else {
#pragma unroll
    for (int c = 0; c < R / CH; ++c) {
      const typename U16Vec<CH>::type q =
          *reinterpret_cast<const typename U16Vec<CH>::type*>(leaf + nid[c * CH]);
#pragma unroll
      for (int u = 0; u < CH; ++u) v[c * CH + u] = q[u];
    }
  }

  // Levels D-1 .. 0: reduce digit k_{m+1}, bits [lo, lo + K) of n.
#pragma unroll
  for (int m = D - 1; m >= 0; --m) {
    const int lo = K * (D - 1 - m), hi = lo + K;
    int rm = ri - 1 - m;
    if (rm < 0) rm += L;
    const f16 wm = f16_bits(wbits[rm]);
    const int nr = lo < RLOG ? R : 1;  // registers still distinct
    const uint32_t hl = tf.level_hash(CB, m);
#pragma unroll
    for (int r = 0; r < nr; ++r) {
      const f16 dh = decode_hash(CB, hl + TreeFields<K, D, RLOG>::level_offset(CB, m, r)) - wm;
      v[r] = bits_f16(__builtin_fmaf16(dh, dh, f16_bits(v[r])));
    }
#pragma unroll
    for (int b = lo; b < (hi < RLOG ? hi : RLOG); ++b)
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (!(r & (1 << b))) {
          const uint32_t t = umin(v[r], v[r | (1 << b)]);
          v[r] = t;
          v[r | (1 << b)] = t;
        }
    if (hi > RLOG) {
#pragma unroll
      for (int b = (lo > RLOG ? lo : RLOG); b < (hi < NLOG ? hi : NLOG); ++b)
        v[0] = xor_min(v[0], 1 << (b - RLOG));
#pragma unroll
      for (int r = 1; r < R; ++r) v[r] = v[0];
    }
  }

  // Step i: key minimum over k_0, bits [K D, NLOG) of n.
  const f16 w = f16_bits(wbits[ri]);
  const int nr = (K * D) < RLOG ? R : 1;
  const uint32_t ht = tf.top_hash(CB, edge);
  uint32_t key = 0xFFFFFFFFu;
#pragma unroll
  for (int r = 0; r < nr; ++r) {
    const uint32_t k0 = nid[r] >> (K * D);
    const f16 dh = decode_hash(CB, ht + TreeFields<K, D, RLOG>::top_offset(CB, r)) - w;
    const f16 err = __builtin_fmaf16(dh, dh, f16_bits(v[r]));
    key = umin(key, ((uint32_t)bits_f16(err) << 16) | k0);
  }
#pragma unroll
  for (int b = (K * D > RLOG ? K * D : RLOG); b < NLOG; ++b)
    key = xor_min(key, 1 << (b - RLOG));
  return key & 0xFFFFu;
}

// The decisions of every step that reads one stored row, from one
// evaluation of the row's depth-D tree. Step i's choice is the key minimum
// at the top; the level-m reduction computes exactly what step i-1-m
// chooses between (the FMA over its 2^K predecessors, whose costs are the
// level below), so if each level reduces keys (cost_bits << 16) | digit
// instead of bare costs, the choice of step i-1-m for the prefix chosen
// above is the digit of the level-m key held by that prefix's lane and
// register (lowest digit on equal costs, as the forward pass). Returns the
// branches packed: bits [K j, K j + K) hold the branch of step i - j,
// j = 0..D (K * row_stride(K) <= 10 bits).
//
// The leaves are read straight from the stored row (HBM, or an LDS copy of
// it): leaf n sits at row_pos(x_D(n)), and a lane's CH leaves that differ
// only in the last digit are one aligned vector of siblings.
template <int K, int CB, int D>
__device__ __forceinline__ uint32_t tb_tree(const uint16_t* __restrict__ row, uint32_t edge,
                                            const uint16_t* __restrict__ wbits, int ri, int L,
                                            int lane) {
  constexpr int NB = 1 << K, KS = 16 - 2 * K;
  constexpr int NLOG = K * (D + 1);
  constexpr int RLOG = NLOG > 6 ? NLOG - 6 : 0;
  constexpr int R = 1 << RLOG;
  constexpr uint32_t NMASK = (1u << NLOG) - 1u;
  // A lane's R leaves are one aligned run in K = 2's tree-major rows, and
  // its 2^K siblings elsewhere.
  constexpr int CH = (K == 2 || K == 3 || R < NB) ? R : NB;
  const uint32_t h0 = edge >> K;

  uint32_t nid[R];
  uint32_t xs[R][D + 1];
  uint32_t v[R];
  TreeFields<K, D, RLOG> tf(lane, h0);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t n = (((uint32_t)lane << RLOG) | (uint32_t)r) & NMASK;
    nid[r] = n;
    uint32_t x = ((n >> (K * D)) << KS) | h0;
    xs[r][0] = x;
#pragma unroll
    for (int m = 1; m <= D; ++m) {
      x = (((n >> (K * (D - m))) & (NB - 1)) << KS) | (x >> K);
      xs[r][m] = x;
    }
  }
#pragma unroll
  for (int c = 0; c < R / CH; ++c) {
    const typename U16Vec<CH>::type q = *reinterpret_cast<const typename U16Vec<CH>::type*>(
        row + row_pos<K>(xs[c * CH][D]));
#pragma unroll
    for (int u = 0; u < CH; ++u) v[c * CH + u] = q[u];
  }
  // A lane's leaves are at most 8 bytes (R <= 4) at every K but 2, whose
  // 16 (32 bytes, two loads) are one aligned run.
  static_assert(R <= 4 || ((K == 2 || K == 3) && R <= 16), "a lane's leaves are one run");

  uint32_t lvl[D > 0 ? D : 1][R];
#pragma unroll
  for (int m = D - 1; m >= 0; --m) {
    const int lo = K * (D - 1 - m), hi = lo + K;
    int rm = ri - 1 - m;
    if (rm < 0) rm += L;
    const f16 wm = f16_bits(wbits[rm]);
    const int nr = lo < RLOG ? R : 1;  // registers still distinct
    const uint32_t hl = tf.level_hash(CB, m);
#pragma unroll
    for (int r = 0; r < nr; ++r) {
      const uint32_t k = (nid[r] >> lo) & (NB - 1);
      const f16 dh = decode_hash(CB, hl + TreeFields<K, D, RLOG>::level_offset(CB, m, r)) - wm;
      v[r] = ((uint32_t)bits_f16(__builtin_fmaf16(dh, dh, f16_bits(v[r]))) << 16) | k;
    }
    if (nr == 1) {
#pragma unroll
      for (int r = 1; r < R; ++r) v[r] = v[0];
    }
#pragma unroll
    for (int b = lo; b < (hi < RLOG ? hi : RLOG); ++b)
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (!(r & (1 << b))) {
          const uint32_t t = umin(v[r], v[r | (1 << b)]);
          v[r] = t;
          v[r | (1 << b)] = t;
        }
    if (hi > RLOG) {
#pragma unroll
      for (int b = (lo > RLOG ? lo : RLOG); b < (hi < NLOG ? hi : NLOG); ++b)
        v[0] = xor_min(v[0], 1 << (b - RLOG));
#pragma unroll
      for (int r = 1; r < R; ++r) v[r] = v[0];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      lvl[m][r] = v[r];
      v[r] >>= 16;
    }
  }

  // Step i: key minimum over k_0, bits [K D, NLOG) of n.
  const f16 w = f16_bits(wbits[ri]);
  const int nr = (K * D) < RLOG ? R : 1;
  const uint32_t ht = tf.top_hash(CB, edge);
  uint32_t key = 0xFFFFFFFFu;
#pragma unroll
  for (int r = 0; r < nr; ++r) {
    const uint32_t k0 = nid[r] >> (K * D);
    const f16 dh = decode_hash(CB, ht + TreeFields<K, D, RLOG>::top_offset(CB, r)) - w;
    const f16 err = __builtin_fmaf16(dh, dh, f16_bits(v[r]));
    key = umin(key, ((uint32_t)bits_f16(err) << 16) | k0);
  }
#pragma unroll
  for (int b = (K * D > RLOG ? K * D : RLOG); b < NLOG; ++b)
    key = xor_min(key, 1 << (b - RLOG));
  uint32_t prefix = (uint32_t)__builtin_amdgcn_readfirstlane((int)key) & 0xFFFFu;
  uint32_t ks = prefix;
#pragma unroll
  for (int m = 0; m < D; ++m) {
    const uint32_t nsel = prefix << (K * (D - m));  // the prefix's first leaf
    const int reg = (int)(nsel & (uint32_t)(R - 1));
    uint32_t sel = lvl[m][0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (r == reg) sel = lvl[m][r];
    const uint32_t kk =
        (uint32_t)__builtin_amdgcn_readlane((int)sel, (int)(nsel >> RLOG)) & 0xFFFFu;
    ks |= kk << (K * (m + 1));
    prefix = (prefix << K) | kk;
  }
  return ks;
}

template <int K, int CB, int D>
__device__ __forceinline__ uint32_t tb_tree_dispatch(int d, const uint16_t* row, uint32_t edge,
                                                     const uint16_t* __restrict__ wbits, int ri,
                                                     int L, int lane) {
  static_assert(K * exl3::row_stride(K) <= 32, "a row's branches fit in one word");
  if constexpr (D + 1 < exl3::row_stride(K)) {
    if (d != D) return tb_tree_dispatch<K, CB, D + 1>(d, row, edge, wbits, ri, L, lane);
  }
  return tb_tree<K, CB, D>(row, edge, wbits, ri, L, lane);
}

// One stored row serves steps i .. r0 + 1: its tree is loaded once, at the
// first of them, and evaluated once (tb_tree), which yields all of their
// branches. One dependent HBM load and one tree evaluation per stride of
// steps.
template <int K, int CB>
__global__ void __launch_bounds__(64) traceback_rows_kernel(TbArgs a) {
  constexpr int KR = 16 - K;
  constexpr int STRIDE = exl3::row_stride(K);
  __shared__ uint16_t s_wbits[256];  // the tile's fp16 inputs, ring order
  __shared__ uint16_t s_oidx[256];   // the walk's states, ring order (write pass)
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const int L = a.L;
  const uint8_t* blk = a.scratch + (int64_t)t * a.tile_stride;
  const uint8_t* hdr = blk + a.hdr_offset;
  const int row_bytes = a.lay.row_bytes;
  const int pre = reinterpret_cast<const int32_t*>(hdr)[exl3::HDR_PRE_STATE];
  const uint16_t* wsrc = reinterpret_cast<const uint16_t*>(hdr + exl3::HDR_W_BYTES);
  for (int r = lane; r < L; r += 64) s_wbits[r] = wsrc[r];
  __syncthreads();
  const uint16_t* wbits = s_wbits;
  uint32_t edge = (uint32_t)a.start[(int64_t)t * a.start_stride] & ((65536u >> K) - 1u);
  const int i_stop = a.write ? 0 : (L - a.roll) % L;  // the last step walked

  int i = L - 1;
  while (i >= 1 && i >= i_stop) {
    // Steps i .. r0 + 1 read stored row r0: one tree load, one evaluation.
    const int d = (i - 1) % STRIDE;
    const int r0 = i - 1 - d;
    const uint16_t* row =
        reinterpret_cast<const uint16_t*>(blk + (int64_t)(r0 / STRIDE) * row_bytes);
    int ri = i + a.roll;
    if (ri >= L) ri -= L;
    const uint32_t ks = tb_tree_dispatch<K, CB, 0>(d, row, edge, wbits, ri, L, lane);
#pragma unroll
    for (int j = 0; j < STRIDE; ++j) {
      if (j <= d && i >= i_stop) {
        int rj = i + a.roll;
        if (rj >= L) rj -= L;
        const uint32_t sigma = (((ks >> (K * j)) & ((1u << K) - 1u)) << KR) | edge;
        if (a.write && lane == 0) s_oidx[rj] = (uint16_t)sigma;
        edge = sigma >> K;
        --i;
      }
    }
  }
  if (i == 0 && i_stop == 0) {  // step 0: predecessors from the start constraint
    int ri = a.roll;
    if (ri >= L) ri -= L;
    const uint32_t k = tb_branch<K, CB, 0, true>(nullptr, edge, wbits, ri, L, lane, pre);
    const uint32_t sigma = (k << KR) | edge;
    if (a.write && lane == 0) s_oidx[ri] = (uint16_t)sigma;
    edge = sigma >> K;
  }
  if (a.write) {
    // The states and their codebook values leave after the walk, coalesced
    // over the wave, so the serial walk carries no decode or global store.
    __syncthreads();
    for (int r = lane; r < L; r += 64) {
      const uint32_t sigma = s_oidx[r];
      a.out_idx[(int64_t)t * L + r] = (int16_t)(uint16_t)sigma;
      a.out_w[(int64_t)t * L + r] = (float)decode_state(CB, sigma);
    }
  } else if (lane == 0) {
    a.end_out[(int64_t)t * a.end_stride] = (int32_t)edge;
  }
}

// Streamed cost-row traceback for small batches. The traceback above is
// bound by one dependent HBM load per stored row and tile; with few tiles
// in flight that latency is the whole kernel. Here one workgroup per tile
// streams every stored row it will visit into a two-slot LDS ring ahead of
// the walk (the rows are known in advance, only the tree inside a row
// depends on the path): wave 0 walks exactly as traceback_rows_kernel,
// reading its trees from the ring; NG loader groups of W waves take rows in
// turn (row j belongs to group j % NG), so a row's load has NG rows of walk
// time to arrive while every group keeps one row in statically indexed
// registers. One workgroup barrier per stored row, LDS-only fences so loads
// stay in flight across it. Reads every row whole (E x 2 bytes instead of
// one tree), so it pays off only while HBM bandwidth is idle.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int K>
struct StreamShape {
  static constexpr int W = (K == 1 || K == 2) ? 4 : (K <= 4 ? 2 : 1);  // waves per group
  static constexpr int NG = (K == 1) ? 1 : (K == 2 ? 2 : (K <= 5 ? 4 : 8));
  static_assert(K >= 1 && K <= 8, "cost-row bitrates");
  static constexpr int THREADS = 64 * (1 + W * NG);
};

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int K, int CB>
__global__ void __launch_bounds__(StreamShape<K>::THREADS) traceback_stream_kernel(TbArgs a) {
  constexpr int KR = 16 - K;
  constexpr int STRIDE = exl3::row_stride(K);
  constexpr int RV = 2 * (65536 >> K) / 16;  // 16-byte vectors per row
  constexpr int W = StreamShape<K>::W, NG = StreamShape<K>::NG;
  constexpr int NLT = 64 * W;                // threads per loader group
  // A row smaller than a loader group (K = 8: 32 vectors) leaves the
  // group's threads lt >= RV idle.
  constexpr bool PART = RV < NLT;
  constexpr int V = PART ? 1 : RV / NLT;
  static_assert(PART || RV % NLT == 0, "rows split evenly over a loader group");
  __shared__ u32x4 s_ring[2][RV];
  __shared__ uint16_t s_wbits[256];
  __shared__ uint16_t s_oidx[256];
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int L = a.L, roll = a.roll;
  const uint8_t* blk = a.scratch + (int64_t)t * a.tile_stride;
  const uint8_t* hdr = blk + a.hdr_offset;
  const int row_bytes = a.lay.row_bytes;
  const int pre = reinterpret_cast<const int32_t*>(hdr)[exl3::HDR_PRE_STATE];
  const uint16_t* wsrc = reinterpret_cast<const uint16_t*>(hdr + exl3::HDR_W_BYTES);
  for (int r = threadIdx.x; r < L; r += StreamShape<K>::THREADS) s_wbits[r] = wsrc[r];

  // Steps L-1 .. i_stop are walked; steps >= 1 read the stored row
  // r0(i) = (i - 1) - (i - 1) % STRIDE, rows top, top - STRIDE, ..., r_last.
  const int i_stop = a.write ? 0 : (L - roll) % L;
  const int last_i = i_stop > 1 ? i_stop : 1;
  const int top = (L - 2) - (L - 2) % STRIDE;
  const int r_last = (last_i - 1) - (last_i - 1) % STRIDE;
  const int NR = (top - r_last) / STRIDE + 1;
  auto row_src = [&](int q) {
    return reinterpret_cast<const u32x4*>(blk + (int64_t)((top - q * STRIDE) / STRIDE) * row_bytes);
  };

  const int g = (wave - 1) / W;              // loader group (wave >= 1)
  const int lt = threadIdx.x - 64 - g * NLT;
  const bool loads = wave > 0 && (!PART || lt < RV);
  u32x4 buf[V];  // native vectors: registers, not scratch
  if (loads) {
    if (g < NR) {
      const u32x4* src = row_src(g);
#pragma unroll
      for (int v = 0; v < V; ++v) buf[v] = src[lt + v * NLT];
    }
    if (g == 0) {
#pragma unroll
      for (int v = 0; v < V; ++v) s_ring[0][lt + v * NLT] = buf[v];
      if (NG < NR) {
        const u32x4* src = row_src(NG);
#pragma unroll
        for (int v = 0; v < V; ++v) buf[v] = src[lt + v * NLT];
      }
    }
  }
  lds_barrier();

  const uint16_t* wbits = s_wbits;
  uint32_t edge = (uint32_t)a.start[(int64_t)t * a.start_stride] & ((65536u >> K) - 1u);
  int i = L - 1;
  for (int q = 0; q < NR; ++q) {
    if (wave == 0) {
      const uint16_t* row = reinterpret_cast<const uint16_t*>(s_ring[q & 1]);
      const int r = top - q * STRIDE;
      if (i >= last_i && (i - 1) - (i - 1) % STRIDE == r) {
        // Steps i .. r + 1 read this row: one tree, one evaluation.
        const int d = (i - 1) % STRIDE;
        int ri = i + roll;
        if (ri >= L) ri -= L;
        const uint32_t ks = tb_tree_dispatch<K, CB, 0>(d, row, edge, wbits, ri, L, lane);
#pragma unroll
        for (int j = 0; j < STRIDE; ++j) {
          if (j <= d && i >= last_i) {
            int rj = i + roll;
            if (rj >= L) rj -= L;
            const uint32_t sigma = (((ks >> (K * j)) & ((1u << K) - 1u)) << KR) | edge;
            if (a.write && lane == 0) s_oidx[rj] = (uint16_t)sigma;
            edge = sigma >> K;
            --i;
          }
        }
      }
    } else if (loads) {
      const int j = q + 1;  // the row to place in the ring this iteration
      if (j < NR && j % NG == g) {
#pragma unroll
        for (int v = 0; v < V; ++v) s_ring[j & 1][lt + v * NLT] = buf[v];
        if (j + NG < NR) {
          const u32x4* src = row_src(j + NG);
#pragma unroll
          for (int v = 0; v < V; ++v) buf[v] = src[lt + v * NLT];
        }
      }
    }
    lds_barrier();
  }

  if (wave != 0) return;
  if (i_stop == 0) {  // step 0: predecessors from the start constraint
    int ri = roll;
    if (ri >= L) ri -= L;
    const uint32_t k = tb_branch<K, CB, 0, true>(nullptr, edge, wbits, ri, L, lane, pre);
    const uint32_t sigma = (k << KR) | edge;
    if (a.write && lane == 0) s_oidx[ri] = (uint16_t)sigma;
    edge = sigma >> K;
  }
  if (a.write) {
    __builtin_amdgcn_wave_barrier();
    for (int r = lane; r < L; r += 64) {
      const uint32_t sigma = s_oidx[r];
      a.out_idx[(int64_t)t * L + r] = (int16_t)(uint16_t)sigma;
      a.out_w[(int64_t)t * L + r] = (float)decode_state(CB, sigma);
    }
  } else if (lane == 0) {
    a.end_out[(int64_t)t * a.end_stride] = (int32_t)edge;
  }
}

// ---------------------------------------------------------- prepare/finalize

// nan_count (may be NULL) gains one per NaN input value, so a caller can
// reject NaN tiles without a device-to-host round trip per batch.
__global__ void prepare_kernel(const float* __restrict__ raw, float* __restrict__ out, int64_t n,
                               int L, int permute, int32_t* __restrict__ nan_count) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * L) return;
  const int64_t t = idx / L;
  const int i = (int)(idx - t * L);
  const float v = raw[t * L + (permute ? tc_perm(i) : i)];
  if (nan_count != nullptr && v != v) atomicAdd(nan_count, 1);
  out[idx] = (float)(f16)v;
}

// numpy float32 pairwise summation (numpy/_core/src/umath/loops_utils.h.src)
// of a block of n in [8, 128] elements from LDS, by the wave: lane j < 8
// accumulates r[j] = a[j] + a[j + 8] + ... in order, the tail n % 8 is
// added after ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)); the xor
// butterfly forms exactly those sums (fp32 addition is commutative). The
// result is valid in lane 0.
__device__ __forceinline__ float pairwise_block_wave(const float* a, int n, int lane) {
  float r = 0.0f;
  if (lane < 8) {
    r = a[lane];
    for (int i = 8; i < n - (n % 8); i += 8) r += a[i + lane];
  }
  r += __shfl_xor(r, 1, 64);
  r += __shfl_xor(r, 2, 64);
  r += __shfl_xor(r, 4, 64);
  for (int i = n - (n % 8); i < n; ++i) r += a[i];
  return r;
}

// np.sum over n in [16, 256] float32 values: 0 + pairwise(n) where blocks
// above 128 split at n/2 rounded down to a multiple of 8.
__device__ __forceinline__ float numpy_sum_f32_wave(const float* a, int n, int lane) {
  if (n <= 128) return 0.0f + pairwise_block_wave(a, n, lane);
  int n2 = n / 2;
  n2 -= n2 % 8;
  const float lo = pairwise_block_wave(a, n2, lane);
  const float hi = pairwise_block_wave(a + n2, n - n2, lane);
  return 0.0f + (lo + hi);
}

// One wave per tile: path cost, distortion, original-order reconstruction
// and packing (reference_encoder.py:296-316, xpu_quantizer.py:933-976).
__global__ void __launch_bounds__(64) finalize_kernel(
    const float* __restrict__ x, const float* __restrict__ raw, const float* __restrict__ out_w,
    const int16_t* __restrict__ out_idx, uint16_t* __restrict__ packed,
    float* __restrict__ path_cost, float* __restrict__ distortion,
    uint16_t* __restrict__ recon_orig, int K, int L, int permuted) {
  __shared__ f16 s_dh[256];
  __shared__ float s_sq[256];
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x;
  const float* xt = x + t * L;
  const float* wt = out_w + t * L;
  const int16_t* it = out_idx + t * L;

  for (int i = lane; i < L; i += 64) {
    s_dh[i] = (f16)wt[i] - (f16)xt[i];
    // Squared error in evaluation order (reference_encoder.py:302-311).
    const int src = permuted ? tc_perm_inv(i) : i;
    const f16 rec = (f16)wt[src];
    if (recon_orig) recon_orig[t * L + i] = bits_f16(rec);
    const float orig = permuted ? raw[t * L + i] : xt[i];
    const float d = orig - (float)rec;
    s_sq[i] = d * d;
  }
  __syncthreads();

  const float dist = numpy_sum_f32_wave(s_sq, L, lane);
  if (lane == 0) {
    distortion[t] = dist;
    // Path cost along the chosen states in ring order (xpu_quantizer.py:933-941).
    f16 acc = __builtin_fmaf16(s_dh[0], s_dh[0], (f16)0);
    for (int i = 1; i < L; ++i) acc = __builtin_fmaf16(s_dh[i], s_dh[i], acc);
    path_cost[t] = (float)acc;
  }

  // pack_trellis + swap16_storage (trellis_format.py:120-174): one span per lane.
  if (packed && L == 256 && lane < 16) {
    uint16_t* o = packed + t * 16 * K;
    const int span = lane;
    uint32_t buf = 0;
    int held = 32, j = span * K;
    for (int e = 0; e < 16; ++e) {
      held -= K;
      buf |= ((uint32_t)(uint16_t)it[span * 16 + e] & ((1u << K) - 1u)) << held;
      if (held <= 16) {
        o[j ^ 1] = (uint16_t)(buf >> 16);  // j ^ 1: half-word swap of each pair
        buf <<= 16;
        held += 16;
        ++j;
      }
    }
  }
}

__global__ void pack_kernel(const int16_t* __restrict__ states, uint16_t* __restrict__ packed,
                            int64_t n, int K) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * 16) return;
  const int64_t t = gid >> 4;
  const int span = (int)(gid & 15);
  const int16_t* it = states + t * 256 + span * 16;
  uint16_t* o = packed + t * 16 * K;
  uint32_t buf = 0;
  int held = 32, j = span * K;
  for (int e = 0; e < 16; ++e) {
    held -= K;
    buf |= ((uint32_t)(uint16_t)it[e] & ((1u << K) - 1u)) << held;
    if (held <= 16) {
      o[j ^ 1] = (uint16_t)(buf >> 16);
      buf <<= 16;
      held += 16;
      ++j;
    }
  }
}

// Inverse of pack_kernel (trellis_format.py:181-213): state t of a tile is
// the 16-bit window of the tile's MSB-first bitstream ending at bit
// (t + 1) K, circular. Stream word w is storage word w ^ 1 (swap16), so the
// window is two neighbouring words shifted; one thread per state.
__global__ void unpack_kernel(const uint16_t* __restrict__ packed, int16_t* __restrict__ states,
                              int64_t n, int K) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * 256) return;
  const int64_t tile = gid >> 8;
  const int t = (int)(gid & 255);
  const int nbits = 256 * K, words = 16 * K;
  const int p0 = ((t + 1) * K - 16 + nbits) % nbits;
  const int w0 = p0 >> 4, off = p0 & 15;
  const uint16_t* src = packed + tile * words;
  const uint32_t hi = src[w0 ^ 1];
  const uint32_t lo = src[((w0 + 1) % words) ^ 1];
  states[gid] = (int16_t)(uint16_t)((((hi << 16) | lo) >> (16 - off)) & 0xFFFFu);
}

__global__ void probe_hfma_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ c,
                                  uint16_t* __restrict__ out, int64_t n, int mode) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const f16 x = f16_bits(a[i]), y = f16_bits(c[i]);
  f16 r;
  if (mode == 0) {
    r = __builtin_fmaf16(x, x, y);
  } else {
    const f16 sq = x * x;  // rounded product (fp-contract is off)
    r = sq + y;
  }
  out[i] = bits_f16(r);
}

// =================================================================== host

static hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------- scratch of the no-alloc entry

// temp_costs then temp_edges of exl3_quantize_tiles_noalloc's tiles. Every
// GPU the library runs on holds its own copy from module load until the
// process ends. Host code never uses this name as an address: it is a
// host-side stand-in, and kernels get the device address that
// hipGetSymbolAddress returns for the current GPU.
__device__ __align__(256) uint8_t scratch[EXL3_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_ptr[kMaxScratchDevices];

// Device address of `scratch` on the calling thread's current GPU, looked
// up once per device with that device current.
static int noalloc_scratch(uint8_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error("quantize_tiles_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error("quantize_tiles_noalloc: device %d outside 0..%d", dev,
                     kMaxScratchDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error("quantize_tiles_noalloc: hipGetSymbolAddress(scratch) failed on device "
                       "%d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

static int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

static int validate_common(int K, int cb, int L) {
  if (K < 1 || K > 8) return set_error("K must be in 1..8, got %d", K);
  if (cb < 0 || cb > 2) return set_error("cb must be 0, 1, or 2, got %d", cb);
  if (L != 256 && L != 160) return set_error("tile length L must be 256 or 160, got %d", L);
  if (L == 160 && cb != 2) return set_error("tile length L=160 is only supported with mul1 (cb=2)");
  return 0;
}

static bool use_generic(int K, int generic) { return generic || !exl3::has_fast_kernel(K); }

static RowLayout layout_for(int K) { return exl3::make_layout(K); }

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int K, int CB>
static void launch_fast_cb(const FwdArgs& a, hipStream_t st) {
  if constexpr (K >= 4) {
    hipLaunchKernelGGL((acs_forward_chunked<K, CB>), dim3(a.n), dim3(1024), 0, st, a);
  } else {
    using Sh = FastShape<K>;
    if (K == 1 && a.n > device_cus()) {
      // More than one workgroup per CU to place: the in-place variant fits two.
      hipLaunchKernelGGL((acs_forward_rows<K, Sh::G, Sh::J, CB, K == 1>), dim3(a.n), dim3(1024), 0,
                         st, a);
      return;
    }
    hipLaunchKernelGGL((acs_forward_rows<K, Sh::G, Sh::J, CB, false>), dim3(a.n), dim3(1024), 0, st,
                       a);
  }
}

template <int K>
static void launch_fast(const FwdArgs& a, hipStream_t st) {
  switch (a.cb) {
    case 0: launch_fast_cb<K, 0>(a, st); break;
    case 1: launch_fast_cb<K, 1>(a, st); break;
    default: launch_fast_cb<K, 2>(a, st); break;
  }
}

static int launch_forward(const FwdArgs& a, int K, int generic, hipStream_t st) {
  if (a.n <= 0) return 0;
  if (use_generic(K, generic)) {
    hipLaunchKernelGGL(acs_forward_generic, dim3(a.n), dim3(GEN_NT), 0, st, a, K);
  } else {
    switch (K) {
      case 1: launch_fast<1>(a, st); break;
      case 2: launch_fast<2>(a, st); break;
      case 3: launch_fast<3>(a, st); break;
      case 4: launch_fast<4>(a, st); break;
      case 5: launch_fast<5>(a, st); break;
      case 6: launch_fast<6>(a, st); break;
      case 7: launch_fast<7>(a, st); break;
      case 8: launch_fast<8>(a, st); break;
      default: return set_error("no fast kernel for K=%d", K);
    }
  }
  return check_launch("acs_forward");
}

static FwdArgs forward_args(const float* in, int n, int K, int cb, int L, uint8_t* scratch,
                            uint16_t* term_costs) {
  const RowLayout lay = layout_for(K);
  FwdArgs a{};
  a.in = in;
  a.n = n;
  a.L = L;
  a.cb = cb;
  a.scratch = scratch;
  a.tile_stride = (int64_t)exl3::tile_scratch_bytes(lay, L);
  a.hdr_offset = exl3::header_offset(lay, L);
  a.term_costs = term_costs;
  a.store_from = 0;
  return a;
}

// Traceback kernel choice: 0 = by batch size, 1 = per-row tree loads
// (traceback_rows_kernel), 2 = streamed rows (traceback_stream_kernel).
// The process default (exl3_set_traceback_policy) applies to calls that do
// not name one; exl3_quantize_tiles_tb takes the choice per call, so two
// threads or streams can choose differently without touching the default.
static std::atomic<int> g_traceback_policy{0};

static int resolve_policy(int policy) {
  return policy < 0 ? g_traceback_policy.load(std::memory_order_relaxed) : policy;
}

// The streamed traceback reads each visited row whole: per row it moves
// tiles x row bytes at the streaming rate, where the per-row walk waits one
// dependent tree load; the walk's row count cancels. Whole encode calls
// measured the crossover at 128-256 tiles for K = 2, 3, about 384 for
// K = 4, about 600 for K = 5 (each 2.5 MiB of rows per step of the walk)
// and above 768 for K = 6..8, where the streamed kernel was 30-110 us per
// call too long at 1024-2048 tiles.
static bool use_stream_traceback(const TbArgs& a, int policy) {
  if (policy == 1) return false;
  if (policy == 2) return true;
  return (int64_t)a.n * a.lay.row_bytes <= ((int64_t)5 << 19) && a.n <= 768;
}

template <int K>
static void launch_traceback_rows(const TbArgs& a, int policy, hipStream_t st) {
  if (use_stream_traceback(a, policy)) {
    const dim3 blk(StreamShape<K>::THREADS);
    switch (a.cb) {
      case 0: hipLaunchKernelGGL((traceback_stream_kernel<K, 0>), dim3(a.n), blk, 0, st, a); break;
      case 1: hipLaunchKernelGGL((traceback_stream_kernel<K, 1>), dim3(a.n), blk, 0, st, a); break;
      default: hipLaunchKernelGGL((traceback_stream_kernel<K, 2>), dim3(a.n), blk, 0, st, a); break;
    }
    return;
  }
  switch (a.cb) {
    case 0: hipLaunchKernelGGL((traceback_rows_kernel<K, 0>), dim3(a.n), dim3(64), 0, st, a); break;
    case 1: hipLaunchKernelGGL((traceback_rows_kernel<K, 1>), dim3(a.n), dim3(64), 0, st, a); break;
    default: hipLaunchKernelGGL((traceback_rows_kernel<K, 2>), dim3(a.n), dim3(64), 0, st, a); break;
  }
}

// policy: 0..2 as above, -1 = the process default.
static int launch_traceback(const TbArgs& a, int policy, hipStream_t st) {
  if (a.n <= 0) return 0;
  const int p = resolve_policy(policy);
  switch (a.lay.K) {
    case 1: launch_traceback_rows<1>(a, p, st); break;
    case 2: launch_traceback_rows<2>(a, p, st); break;
    case 3: launch_traceback_rows<3>(a, p, st); break;
    case 4: launch_traceback_rows<4>(a, p, st); break;
    case 5: launch_traceback_rows<5>(a, p, st); break;
    case 6: launch_traceback_rows<6>(a, p, st); break;
    case 7: launch_traceback_rows<7>(a, p, st); break;
    default: launch_traceback_rows<8>(a, p, st); break;
  }
  return check_launch("traceback");
}

static TbArgs traceback_args(const uint8_t* scratch, int n, int K, int cb, int L, int roll,
                             int write) {
  const RowLayout lay = layout_for(K);
  TbArgs t{};
  t.scratch = scratch;
  t.tile_stride = (int64_t)exl3::tile_scratch_bytes(lay, L);
  t.hdr_offset = exl3::header_offset(lay, L);
  t.lay = lay;
  t.n = n;
  t.L = L;
  t.roll = roll;
  t.write = write;
  t.cb = cb;
  return t;
}

extern "C" {

const char* exl3_last_error(void) { return g_last_error.c_str(); }

const char* exl3_version(void) { return EXL3_VERSION; }

int exl3_set_traceback_policy(int policy) {
  if (policy < 0 || policy > 2)
    return set_error("traceback policy must be 0, 1 or 2, got %d", policy), -1;
  return g_traceback_policy.exchange(policy);
}

int exl3_decode_codebook(int cb, uint16_t* lut, void* stream) {
  if (cb < 0 || cb > 2) return set_error("cb must be 0, 1, or 2, got %d", cb);
  if (!lut) return set_error("lut must not be NULL");
  hipLaunchKernelGGL(decode_codebook_kernel, dim3(256), dim3(256), 0, as_stream(stream), cb, lut);
  return check_launch("decode_codebook");
}

int64_t exl3_scratch_row_bytes(int K) {
  if (K < 1 || K > 8) return set_error("K must be in 1..8, got %d", K), -1;
  return layout_for(K).row_bytes;
}

int64_t exl3_scratch_edges_bytes(int K, int L, int64_t tiles) {
  if (K < 1 || K > 8 || L <= 0 || tiles < 0) return set_error("bad scratch arguments"), -1;
  return (int64_t)exl3::tile_scratch_bytes(layout_for(K), L) * tiles;
}

int64_t exl3_cost_row_slot(int K, int64_t edge) {
  if (K < 1 || K > 8 || edge < 0 || edge >= (65536 >> K)) return set_error("bad edge"), -1;
  return exl3::row_slot(layout_for(K), (uint32_t)edge);
}

int exl3_forward_pass(const float* in, uint16_t* temp_costs, uint8_t* temp_edges,
                      const int32_t* pre_states, int64_t n, int K, int cb, int L, int roll,
                      int cost_slot, int generic, void* stream) {
  if (validate_common(K, cb, L)) return 1;
  if (n <= 0 || n > INT32_MAX) return set_error("num_tiles must be positive, got %lld", (long long)n);
  if (cost_slot != 0 && cost_slot != 1) return set_error("cost_slot must be 0 or 1");
  if (roll < 0 || roll >= L) return set_error("roll must be in [0, L), got %d", roll);
  if (!in || !temp_costs || !temp_edges || !pre_states) return set_error("NULL buffer");
  FwdArgs a = forward_args(in, (int)n, K, cb, L, temp_edges, temp_costs);
  a.roll = roll;
  a.pre_states = pre_states;
  a.pre_stride = 1;
  a.cost_slot = cost_slot;
  return launch_forward(a, K, generic, as_stream(stream));
}

int exl3_backward_pass(const uint16_t* temp_costs, const uint8_t* temp_edges, float* out_w,
                       int16_t* out_idx, int32_t* end_states, int64_t n, int K, int cb, int L,
                       int roll, int cost_slot, int write, void* stream) {
  if (validate_common(K, cb, L)) return 1;
  if (n <= 0 || n > INT32_MAX) return set_error("num_tiles must be positive, got %lld", (long long)n);
  if (cost_slot != 0 && cost_slot != 1) return set_error("cost_slot must be 0 or 1");
  if (roll < 0 || roll >= L) return set_error("roll must be in [0, L), got %d", roll);
  if (!temp_costs || !temp_edges || !end_states) return set_error("NULL buffer");
  if (write && (!out_w || !out_idx)) return set_error("NULL output buffer");
  hipStream_t st = as_stream(stream);
  TbArgs t = traceback_args(temp_edges, (int)n, K, cb, L, roll, write);
  t.start = end_states;
  t.start_stride = 1;
  if (!write) {
    const int E = 65536 >> K;
    hipLaunchKernelGGL(argmin_costs_kernel, dim3((unsigned)n), dim3(256), 0, st, temp_costs, E,
                       cost_slot, end_states);
    if (check_launch("argmin_costs")) return 1;
    t.end_out = end_states;
    t.end_stride = 1;
  } else {
    t.out_w = out_w;
    t.out_idx = out_idx;
  }
  return launch_traceback(t, -1, st);
}

int exl3_quantize_tiles_tb(const float* in, float* out_w, int16_t* out_idx,
                           uint16_t* temp_costs, uint8_t* temp_edges, int64_t batch_cap,
                           int64_t n, int K, int cb, int L, int generic, int64_t wave_cap,
                           int traceback, void* stream) {
  if (validate_common(K, cb, L)) return 1;
  if (traceback < -1 || traceback > 2)
    return set_error("traceback must be -1, 0, 1 or 2, got %d", traceback);
  if (n <= 0) return set_error("num_tiles must be positive, got %lld", (long long)n);
  if (batch_cap < 1) return set_error("temp_costs batch dimension B must be >= 1");
  if (!in || !out_w || !out_idx || !temp_costs || !temp_edges) return set_error("NULL buffer");
  const RowLayout lay = layout_for(K);
  const int64_t stride = (int64_t)exl3::tile_scratch_bytes(lay, L);
  // Header row of each tile: int32 {pass-1 terminal edge, end state, ...}.
  const int64_t hstride = stride / 4;
  int32_t* hdr = reinterpret_cast<int32_t*>(temp_edges + exl3::header_offset(lay, L));
  int32_t* best_edges = hdr + exl3::HDR_BEST_EDGE;
  int32_t* end_states = hdr + exl3::HDR_END_STATE;
  const int64_t cap = (wave_cap > 0) ? std::min(batch_cap, wave_cap) : batch_cap;
  const int64_t chunk_max = std::min<int64_t>(cap, INT32_MAX);
  hipStream_t st = as_stream(stream);

  for (int64_t off = 0; off < n; off += chunk_max) {
    const int chunk = (int)std::min<int64_t>(chunk_max, n - off);
    FwdArgs a = forward_args(in + off * L, chunk, K, cb, L, temp_edges, temp_costs);
    // Pass 1: rotation L/2, unconstrained. The traceback covers ring rows
    // 0..L/2-1 only, i.e. forward steps L/2..L-1 (reference_encoder.py:284-288),
    // so only the cost rows those steps need are stored.
    a.roll = L / 2;
    a.store_from = exl3::first_needed_row(lay, L);
    a.cost_slot = 0;
    a.best_edges = best_edges;
    a.best_stride = hstride;
    if (launch_forward(a, K, generic, st)) return 1;
    TbArgs t1 = traceback_args(temp_edges, chunk, K, cb, L, L / 2, 0);
    t1.start = best_edges;
    t1.start_stride = hstride;
    t1.end_out = end_states;
    t1.end_stride = hstride;
    if (launch_traceback(t1, traceback, st)) return 1;
    // Pass 2: natural order, wrap constrained to the end state (:290-293).
    a.roll = 0;
    a.store_from = 0;
    a.pre_states = end_states;
    a.pre_stride = hstride;
    a.cost_slot = 1;
    a.best_edges = nullptr;
    if (launch_forward(a, K, generic, st)) return 1;
    TbArgs t2 = traceback_args(temp_edges, chunk, K, cb, L, 0, 1);
    t2.start = end_states;
    t2.start_stride = hstride;
    t2.out_w = out_w + off * L;
    t2.out_idx = out_idx + off * L;
    if (launch_traceback(t2, traceback, st)) return 1;
  }
  return 0;
}

int exl3_quantize_tiles(const float* in, float* out_w, int16_t* out_idx, uint16_t* temp_costs,
                        uint8_t* temp_edges, int64_t batch_cap, int64_t n, int K, int cb, int L,
                        int generic, int64_t wave_cap, void* stream) {
  return exl3_quantize_tiles_tb(in, out_w, out_idx, temp_costs, temp_edges, batch_cap, n, K, cb,
                                L, generic, wave_cap, -1, stream);
}

int exl3_quantize_tiles_noalloc(const float* in, float* out_w, int16_t* out_idx, int64_t n,
                                int K, int cb, int L, int generic, void* stream) {
  if (validate_common(K, cb, L)) return 1;
  if (n <= 0) return set_error("num_tiles must be positive, got %lld", (long long)n);
  if (!in || !out_w || !out_idx) return set_error("NULL buffer");
  // Per tile: 2 x E fp16 terminal costs and one tile block of temp_edges.
  const int64_t costs_per_tile = 4 * (int64_t)(65536 >> K);
  const int64_t edges_per_tile = (int64_t)exl3::tile_scratch_bytes(layout_for(K), L);
  const int64_t limit = EXL3_NOALLOC_SCRATCH_BYTES;
  const int64_t max_tiles = (limit - 255) / (costs_per_tile + edges_per_tile);
  if (n > max_tiles)
    return set_error("quantize_tiles_noalloc: %lld tiles exceed the %lld-byte static scratch, "
                     "which holds at most %lld tiles at K=%d, L=%d; split the batch",
                     (long long)n, (long long)limit, (long long)max_tiles, K, L);
  uint8_t* base = nullptr;
  if (noalloc_scratch(&base)) return 1;
  uint16_t* temp_costs = reinterpret_cast<uint16_t*>(base);
  uint8_t* temp_edges = base + align256(n * costs_per_tile);
  // Every scratch byte a kernel reads was written earlier in the same call,
  // so nothing is cleared.
  return exl3_quantize_tiles(in, out_w, out_idx, temp_costs, temp_edges, n, n, K, cb, L, generic,
                             0, stream);
}

int exl3_prepare_tiles(const float* raw, float* out, int64_t n, int L, int permute,
                       int32_t* nan_count, void* stream) {
  if (n <= 0 || L <= 0) return set_error("bad tile batch shape");
  if (permute && L != 256) return set_error("pre_permute=True is only defined for L=256");
  if (!raw || !out) return set_error("NULL buffer");
  const int block = 256;
  unsigned blocks;
  if (grid_1d(n * L, block, &blocks, "prepare_tiles")) return 1;
  hipLaunchKernelGGL(prepare_kernel, dim3(blocks), dim3(block), 0, as_stream(stream), raw, out, n,
                     L, permute, nan_count);
  return check_launch("prepare_tiles");
}

int exl3_finalize_tiles(const float* x, const float* raw, const float* out_w,
                        const int16_t* out_idx, uint16_t* packed, float* path_cost,
                        float* distortion, uint16_t* recon_orig, int64_t n, int K, int L,
                        int permuted, void* stream) {
  if (n <= 0 || K < 1 || K > 8 || (L != 256 && L != 160)) return set_error("bad finalize shape");
  if (permuted && (L != 256 || !raw)) return set_error("permuted finalize needs L=256 raw tiles");
  if (!x || !out_w || !out_idx || !path_cost || !distortion) return set_error("NULL buffer");
  if (n > INT32_MAX) return set_error("too many tiles for one finalize launch");
  hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)n), dim3(64), 0, as_stream(stream), x, raw,
                     out_w, out_idx, packed, path_cost, distortion, recon_orig, K, L, permuted);
  return check_launch("finalize_tiles");
}

int exl3_pack_trellis(const int16_t* states, uint16_t* packed, int64_t n, int K, void* stream) {
  if (n <= 0 || K < 1 || K > 8) return set_error("bad pack arguments");
  if (!states || !packed) return set_error("NULL buffer");
  const int block = 256;
  unsigned blocks;
  if (grid_1d(n * 16, block, &blocks, "pack_trellis")) return 1;
  hipLaunchKernelGGL(pack_kernel, dim3(blocks), dim3(block), 0, as_stream(stream), states, packed,
                     n, K);
  return check_launch("pack_trellis");
}

int exl3_unpack_trellis(const uint16_t* packed, int16_t* states, int64_t n, int K, void* stream) {
  if (n <= 0 || K < 1 || K > 8) return set_error("bad unpack arguments");
  if (!packed || !states) return set_error("NULL buffer");
  const int block = 256;
  unsigned blocks;
  if (grid_1d(n * 256, block, &blocks, "unpack_trellis")) return 1;
  hipLaunchKernelGGL(unpack_kernel, dim3(blocks), dim3(block), 0, as_stream(stream), packed,
                     states, n, K);
  return check_launch("unpack_trellis");
}

int exl3_probe_hfma(const uint16_t* a, const uint16_t* c, uint16_t* out, int64_t n, int mode,
                    void* stream) {
  if (n <= 0) return set_error("n must be positive");
  if (mode != 0 && mode != 1) return set_error("mode must be 0 or 1, got %d", mode);
  if (!a || !c || !out) return set_error("NULL buffer");
  const int block = 256;
  unsigned blocks;
  if (grid_1d(n, block, &blocks, "probe_hfma")) return 1;
  hipLaunchKernelGGL(probe_hfma_kernel, dim3(blocks), dim3(block), 0, as_stream(stream), a, c, out,
                     n, mode);
  return check_launch("probe_hfma");
}

}  // extern "C"
