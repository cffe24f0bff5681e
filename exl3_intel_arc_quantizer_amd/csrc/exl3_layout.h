// Trellis geometry and per-tile scratch layout shared by the HIP kernels and
// the host side of the C-ABI.
//
// Trellis (reference: exl3_quant/reference_encoder.py:89-113,
// docs/algorithm_contract.md:199-213). A 16-bit state sigma at bitrate K is
// written sigma = (k << (16-K)) | e with branch k in [0, 2^K) and edge
// e in [0, E), E = 2^(16-K). Its predecessor edge is sigma >> K.
// Writing e = (h << K) | j with group h in [0, S), S = 2^(16-2K), and
// j in [0, 2^K), the predecessor is (k << (16-2K)) | h: all 2^K edges of
// group h read the same 2^K predecessor costs. That 2^K x 2^K block is the
// unit of work the fast kernels assign to threads.
//
// The reference keeps, per (ring row, edge), the chosen predecessor edge as
// int16 (quantize_kernels.sycl:124,153). Here the per-tile scratch holds one
// of two things, chosen by K:
//
// * backpointer rows (K = 1, 2, 8): only the winning branch k, in BPB bits
//   per edge (K rounded up to 1, 2, 4 or 8), since the predecessor is
//   (k << (16-2K)) | (e >> K). Inside a row the fields are in "slot" order:
//   the fast kernel's thread `unit` owns G*J consecutive slots and writes
//   them with one 32-bit store per step; bp_slot() maps an edge to its slot.
//   Row r holds ring row r.
// * cost rows (K = 3..7): the fp16 path-cost vector after a step (E * 2
//   bytes). The forward pass then only needs the minimum cost per edge, which
//   packed fp16 arithmetic computes at the VALU roofline, and the traceback
//   recomputes the 2^K candidates of the one edge on the path from row i-1
//   (the costs the forward step i read). Row i holds the output of trellis
//   step i (step order, independent of the ring roll). A row is group-major:
//   predecessor edge x = (k << (16-2K)) | h sits at position (h << K) | k,
//   so the 2^K costs one traceback step reads are one contiguous chunk. At
//   K = 3..5 only even steps are stored (the rows are 16-64 KiB of HBM
//   writes per step); for an odd row the traceback recomputes the 2^K
//   costs it needs, each a minimum over 2^K candidates from the chunk of
//   row i-2 that the forward pass read. For K <= 2 rows would outweigh the
//   HBM budget (32-64 KiB/step).
//
// Per-tile block: (L + 1) rows of row_bytes. Row L is a header:
//   int32 [0] pass-1 terminal edge, [1] end state, [2] pre_state of the last
//   forward pass; from byte 16, L fp16 inputs in ring order (cost-row mode),
//   which the traceback reads.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define EXL3_HD __host__ __device__
#else
#define EXL3_HD
#endif

namespace exl3 {

enum { MODE_BACKPOINTERS = 0, MODE_COST_ROWS = 1 };

struct BpLayout {
  int32_t K;        // bitrate
  int32_t mode;     // MODE_BACKPOINTERS or MODE_COST_ROWS
  int32_t G;        // groups per thread (backpointer slot order)
  int32_t J;        // edges per group per thread (backpointer slot order)
  int32_t BPB;      // bits per field (16 in cost-row mode)
  int32_t natural;  // 1: slot == edge
  int32_t row_bytes;
};

EXL3_HD inline bool uses_cost_rows(int K) { return K >= 3 && K <= 7; }

EXL3_HD inline int32_t bits_per_backpointer(int K) {
  return K == 3 ? 4 : (K >= 5 ? 8 : K);
}

// Thread decomposition of the fast forward kernels for each K (all use 1024
// threads and 64 candidate branches per thread per step). A thread owns J
// edges of each of G groups, processed in packed pairs (j, j + 1); P lanes
// split the 2^K branches of one edge set, Q = 2^K / P per lane:
//   K : G  J  P   Q   scratch
//   1 : 16 2  1   2   backpointers (tournament kernel)
//   2 :  4 4  1   4   backpointers (tournament kernel)
//   3 :  1 8  1   8   cost rows (row kernel)
//   4 :  1 4  1  16   cost rows
//   5 :  1 2  1  32   cost rows
//   6 :  1 2  2  32   cost rows
//   7 :  1 2  4  32   cost rows
// K = 8 has a single group and runs on the generic kernel. Must match
// FastShape in exl3_encoder.hip.
EXL3_HD inline int fast_G(int K) { return K == 1 ? 16 : (K == 2 ? 4 : 1); }
EXL3_HD inline int fast_J(int K) {
  return K == 1 ? 2 : (K == 2 ? 4 : (K == 3 ? 8 : (K == 4 ? 4 : 2)));
}
EXL3_HD inline int fast_P(int K) { return K == 6 ? 2 : (K == 7 ? 4 : 1); }
EXL3_HD inline bool has_fast_kernel(int K) { return K >= 1 && K <= 7; }

// Scratch layout of bitrate K (the same for every kernel variant, so the
// split forward/backward passes may mix them).
EXL3_HD inline BpLayout make_layout(int K) {
  BpLayout l;
  l.K = K;
  const int E = 65536 >> K;
  l.mode = uses_cost_rows(K) ? MODE_COST_ROWS : MODE_BACKPOINTERS;
  l.G = fast_G(K);
  l.J = fast_J(K);
  l.natural = (K == 8) ? 1 : 0;
  if (l.mode == MODE_COST_ROWS) {
    l.BPB = 16;
    l.row_bytes = E * 2;
  } else {
    l.BPB = (K == 8) ? 8 : bits_per_backpointer(K);
    l.row_bytes = E * l.BPB / 8;
  }
  return l;
}

// Cost rows: which steps are stored, and where edge x sits in a row.
EXL3_HD inline bool sparse_cost_rows(int K) { return K >= 3 && K <= 5; }
EXL3_HD inline bool cost_row_stored(int K, int step) {
  return !sparse_cost_rows(K) || (step & 1) == 0;
}
EXL3_HD inline uint32_t cost_row_pos(int K, uint32_t x) {
  const int ks = 16 - 2 * K;
  return ((x & ((1u << ks) - 1u)) << K) | (x >> ks);
}
// First row the pass-1 traceback reaches (it covers steps L-1 .. L/2 and
// reads rows L/2-1 .. L-2; an odd row needs the even row before it).
EXL3_HD inline int first_needed_row(int K, int L) {
  const int r = L / 2 - 1;
  return sparse_cost_rows(K) ? (r & ~1) : r;
}

// Slot of edge e inside a scratch row: cost_row_pos in cost-row mode.
// Thread `unit` of the tournament kernel owns all 2^K edges of groups
// h0 .. h0 + G - 1 and one 32-bit word per row. Its packed register pair
// pp = g * (J / 2) + (j >> 1) holds edges j (low half, hf = 0) and j + 1
// (high half, hf = 1) of group h0 + g, j even. The kernel gathers pairs 2c
// and 2c + 1 into the four bytes of one word (byte 2u + hf for pair 2c + u)
// and stacks the c-th word at bit K * c of every byte, so the field of an
// edge starts at bit 8 (2u + hf) + K c of the word.
EXL3_HD inline uint32_t bp_slot(const BpLayout& l, uint32_t e) {
  if (l.mode == MODE_COST_ROWS) return cost_row_pos(l.K, e);
  if (l.natural) return e;
  const uint32_t h = e >> l.K;
  const uint32_t j = e & ((1u << l.K) - 1u);
  const uint32_t G = (uint32_t)l.G, J = (uint32_t)l.J;
  const uint32_t NJ = (1u << l.K) / J;
  const uint32_t unit = (h / G) * NJ + j / J;
  const uint32_t jl = j % J;
  const uint32_t pp = (h % G) * (J / 2u) + (jl >> 1);
  const uint32_t bit = 8u * (2u * (pp & 1u) + (jl & 1u)) + (uint32_t)l.K * (pp >> 1);
  return unit * (G * J) + bit / (uint32_t)l.K;
}

EXL3_HD inline uint64_t tile_scratch_bytes(const BpLayout& l, int L) {
  return (uint64_t)(L + 1) * (uint64_t)l.row_bytes;
}

// Header row fields (row L of each tile block).
constexpr int HDR_BEST_EDGE = 0;  // int32 index
constexpr int HDR_END_STATE = 1;  // int32 index
constexpr int HDR_PRE_STATE = 2;  // int32 index
constexpr int HDR_W_BYTES = 16;   // byte offset of the L fp16 inputs (cost-row mode)

}  // namespace exl3
