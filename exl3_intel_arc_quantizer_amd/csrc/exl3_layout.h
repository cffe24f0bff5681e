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
// unit of work the forward kernels assign to threads.
//
// The reference keeps, per (ring row, edge), the chosen predecessor edge as
// int16 (quantize_kernels.sycl:124,153). Here the per-tile scratch holds
// cost rows at every K = 1..8:
//
// * the fp16 path-cost vector after a step (E * 2
//   bytes). The forward pass then only needs the minimum cost per edge, which
//   packed fp16 arithmetic computes at the VALU roofline, and the traceback
//   recomputes the 2^K candidates of the one edge on the path from the costs
//   of step i-1 (the costs the forward step i read). A row is group-major:
//   predecessor edge x = (k << (16-2K)) | h sits at position (h << K) | k,
//   so the 2^K costs one traceback step reads are one contiguous chunk
//   (K = 4 also keeps part of the digit before beside it, and K = 2, 3 keep
//   whole traceback trees together, see cost_row_pos).
//   Only every row_stride(K)-th step is stored (8 KiB or less of HBM writes
//   per step at K <= 5, every step at K >= 6, where a row is 2 KiB or less);
//   for a step d rows past the last stored one, the
//   traceback rebuilds the costs it needs level by level, each a minimum
//   over 2^K candidates, from 2^(K(d+1)) entries of the stored row. Stored
//   step r sits in row slot r / stride, in step order (independent of the
//   ring roll).
//
// Per-tile block: tile_rows(K, L) rows of row_bytes: the stored rows, then
// the header (one row, two at K = 8 where a row is 512 bytes): int32 [0]
// pass-1 terminal edge, [1] end state, [2] pre_state of the last forward
// pass; from byte 16, the L fp16 inputs in ring order, which the traceback
// reads.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define EXL3_HD __host__ __device__
#else
#define EXL3_HD
#endif

namespace exl3 {

struct RowLayout {
  int32_t K;          // bitrate
  int32_t stride;     // every stride-th step's cost row is stored
  int32_t row_bytes;  // E fp16 costs
  int32_t reserved;
};

// Steps between stored cost rows: 8 KiB of HBM writes per step at K = 1,
// 6.4 KiB at K = 2, 5.3 KiB at K = 3, 4 KiB at K = 4, every step at K >= 5
// (where a row is 4 KiB or less). At K = 5 every-step rows double the
// forward pass's writes but cut the traceback's trees from 1024 costs to
// 32: a whole encode is faster at every batch size (8192 tiles -2 %, 256
// tiles -6 %). At K = 2 stride 5 and at K = 3 stride 3 (trees of 1024 and
// 512 costs, each kept whole by a tree-major row layout) write 20 % and
// 33 % less than strides 4 and 2: whole encodes -1 to -2.4 % (K = 2) and
// -2.5 to -8.3 % (K = 3) at 256-8192 tiles.
EXL3_HD constexpr inline int row_stride(int K) {
  return K == 1 ? 8 : (K == 2 ? 5 : (K == 3 ? 3 : (K == 4 ? 2 : 1)));
}

// The fast forward kernels cover K = 1..8: an edge-order kernel for K = 1..3
// and a chunk-major one for K = 4..8 (their thread decompositions are in
// exl3_encoder.hip). Both write the same scratch layout.
EXL3_HD inline bool has_fast_kernel(int K) { return K >= 1 && K <= 8; }

// Scratch layout of bitrate K (the same for every kernel variant, so the
// split forward/backward passes may mix them).
EXL3_HD inline RowLayout make_layout(int K) {
  RowLayout l;
  l.K = K;
  l.stride = row_stride(K);
  l.row_bytes = (65536 >> K) * 2;
  l.reserved = 0;
  return l;
}

// Which steps are stored, where, and where edge x sits in a row.
EXL3_HD inline bool cost_row_stored(const RowLayout& l, int step) { return step % l.stride == 0; }
EXL3_HD inline int cost_row_slot(const RowLayout& l, int step) { return step / l.stride; }
// Group-major: x = (k << (16-2K)) | h at (h << K) | k, so the 2^K costs a
// traceback step compares are one chunk. At K = 4, where a stored row
// serves two steps and one traceback tree spans 2^(2K) entries, the row
// also keeps part of the digit before k beside it: the last digit
// (x >> (16-2K)) at positions [0, K), then the lowest cost_row_tree_bits(K)
// bits of the digit before it, then the other bits of x from bit 1 up, and
// x bit 0 on top. A tree then covers 4 cache lines instead of 16.
//
// K = 2 (stride 5) and K = 3 (stride 3) are tree-major: position bit j holds
// edge bit kRowBitsK2[j] / kRowBitsK3[j]. The edge bits a traceback tree
// spans (x4..x13 at K = 2, x4..x12 at K = 3) are the low positions, last
// digit first, so a tree is one aligned run of 1024 / 512 positions (2 KiB
// or 1 KiB; the group-major order spread a K = 2 tree over 64 cache lines);
// the fixed bits x1..x3 follow and x0 is on top, so the edge-order LDS
// neighbours x, x + 1 sit at positions t, t + E/2 (one dword, two pieces,
// for the forward pass's gather). That gather keeps its LDS reads
// conflict-free by giving each half-wave pieces that differ in x1..x5
// (RowGather).
EXL3_HD constexpr inline int cost_row_tree_bits(int K) {
  return K == 2 ? 10 : (K == 3 ? 9 : (K == 4 ? 2 : 0));
}
constexpr int kRowBitsK2[14] = {12, 13, 10, 11, 4, 5, 6, 7, 8, 9, 1, 2, 3, 0};
constexpr int kRowBitsK3[13] = {10, 11, 12, 4, 5, 6, 7, 8, 9, 1, 2, 3, 0};
EXL3_HD inline uint32_t cost_row_pos(int K, uint32_t x) {
  if (K == 2) {
    uint32_t t = 0;
    for (int j = 0; j < 14; ++j) t |= ((x >> kRowBitsK2[j]) & 1u) << j;
    return t;
  }
  if (K == 3) {
    uint32_t t = 0;
    for (int j = 0; j < 13; ++j) t |= ((x >> kRowBitsK3[j]) & 1u) << j;
    return t;
  }
  const int ks = 16 - 2 * K;
  const int a = cost_row_tree_bits(K);
  if (a == 0) return ((x & ((1u << ks) - 1u)) << K) | (x >> ks);
  const int kb = 16 - K, lo = ks - K;
  const uint32_t rest = ((x >> 1) & ((1u << (lo - 1)) - 1u)) |
                        (((x >> (lo + a)) & ((1u << (ks - lo - a)) - 1u)) << (lo - 1));
  return (x >> ks) | (((x >> lo) & ((1u << a) - 1u)) << K) | (rest << (K + a)) |
         ((x & 1u) << (kb - 1));
}
// The edge at position t of a stored row (the inverse of cost_row_pos).
EXL3_HD inline uint32_t cost_row_edge(int K, uint32_t t) {
  if (K == 2) {
    uint32_t x = 0;
    for (int j = 0; j < 14; ++j) x |= ((t >> j) & 1u) << kRowBitsK2[j];
    return x;
  }
  if (K == 3) {
    uint32_t x = 0;
    for (int j = 0; j < 13; ++j) x |= ((t >> j) & 1u) << kRowBitsK3[j];
    return x;
  }
  const int ks = 16 - 2 * K;
  const int a = cost_row_tree_bits(K);
  if (a == 0) return ((t & ((1u << K) - 1u)) << ks) | (t >> K);
  const int kb = 16 - K, lo = ks - K;
  const uint32_t rest = (t >> (K + a)) & ((1u << (ks - 1 - a)) - 1u);
  return ((t & ((1u << K) - 1u)) << ks) | (((t >> K) & ((1u << a) - 1u)) << lo) |
         ((rest & ((1u << (lo - 1)) - 1u)) << 1) | ((rest >> (lo - 1)) << (lo + a)) |
         (t >> (kb - 1));
}
// First row the pass-1 traceback reaches: it covers steps L-1 .. L/2 and
// needs the stored row at or before L/2 - 1.
EXL3_HD inline int first_needed_row(const RowLayout& l, int L) {
  const int r = L / 2 - 1;
  return r - r % l.stride;
}

// Header row fields.
constexpr int HDR_BEST_EDGE = 0;  // int32 index
constexpr int HDR_END_STATE = 1;  // int32 index
constexpr int HDR_PRE_STATE = 2;  // int32 index
constexpr int HDR_W_BYTES = 16;   // byte offset of the L fp16 inputs

// Stored rows per tile: steps 0, stride, ..., up to L - 2 (the traceback
// never reads the costs after the last step).
EXL3_HD inline int stored_rows(const RowLayout& l, int L) { return (L - 2) / l.stride + 1; }

// Header rows: the 16-byte fields and the L fp16 inputs.
EXL3_HD inline int header_rows(const RowLayout& l, int L) {
  return (HDR_W_BYTES + 2 * L + l.row_bytes - 1) / l.row_bytes;
}

EXL3_HD inline int tile_rows(const RowLayout& l, int L) {
  return stored_rows(l, L) + header_rows(l, L);
}

EXL3_HD inline uint64_t tile_scratch_bytes(const RowLayout& l, int L) {
  return (uint64_t)tile_rows(l, L) * (uint64_t)l.row_bytes;
}

// Byte offset of the header inside a tile block.
EXL3_HD inline int64_t header_offset(const RowLayout& l, int L) {
  return (int64_t)stored_rows(l, L) * l.row_bytes;
}

// Position of edge e inside a stored row.
EXL3_HD inline uint32_t row_slot(const RowLayout& l, uint32_t e) { return cost_row_pos(l.K, e); }

// tensor_core_perm (reference trellis_format.py:88-108): encoded element
// 8t + s is original position row*16 + col with row in
// {2(t%4), 2(t%4)+1, 2(t%4)+8, 2(t%4)+9}[s%4] and col = t/4 + 8*(s/4).
EXL3_HD inline int tc_perm(int i) {
  const int t = i >> 3, s = i & 7;
  const int r0 = (t & 3) * 2;
  const int row = r0 + (s & 1) + ((s >> 1) & 1) * 8;
  const int col = (t >> 2) + (s >> 2) * 8;
  return row * 16 + col;
}

// Inverse of tc_perm: original position p -> encoded element.
EXL3_HD inline int tc_perm_inv(int p) {
  const int row = p >> 4, col = p & 15;
  const int t = ((col & 7) << 2) | ((row & 7) >> 1);
  const int s = (row & 1) | ((row >> 3) << 1) | ((col >> 3) << 2);
  return (t << 3) | s;
}

}  // namespace exl3
