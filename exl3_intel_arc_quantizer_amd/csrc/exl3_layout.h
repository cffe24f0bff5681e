// Trellis geometry and backpointer layout shared by the HIP kernels and the
// host side of the C-ABI.
//
// Trellis (reference: exl3_quant/reference_encoder.py:89-113,
// docs/algorithm_contract.md:199-213). A 16-bit state sigma at bitrate K is
// written sigma = (k << (16-K)) | e with branch k in [0, 2^K) and edge
// e in [0, E), E = 2^(16-K). Its predecessor edge is sigma >> K.
// Writing e = (h << K) | j with group h in [0, S), S = 2^(16-2K), and
// j in [0, 2^K), the predecessor is (k << (16-2K)) | h: all 2^K edges of
// group h read the same 2^K predecessor costs. That 2^K x 2^K block is the
// unit of work the fast kernel assigns to threads.
//
// Backpointers. The reference stores the full predecessor edge as int16 per
// (ring row, edge) (quantize_kernels.sycl:124,153). Here only the winning
// branch k is stored, in BPB bits per edge (BPB = K rounded up to 1, 2, 4 or
// 8 so that fields never straddle a byte boundary), since the predecessor
// is (k << (16-2K)) | (e >> K). Inside a row the fields are stored in
// "slot" order: the fast kernel's thread `unit` owns EPT = G*J consecutive
// slots, so each thread writes its bits for a step with one 16- or 32-bit
// store. bp_slot() maps an edge to its slot.
//
// Per-tile scratch block: (L + 1) rows of ROWB = E*BPB/8 bytes. Rows 0..L-1
// hold the backpointers of ring rows 0..L-1; row L is a header holding
// int32 {pass-1 terminal edge, end state} for the fused encoder.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define EXL3_HD __host__ __device__
#else
#define EXL3_HD
#endif

namespace exl3 {

struct BpLayout {
  int32_t K;        // bitrate
  int32_t G;        // groups per thread (fast layout)
  int32_t J;        // edges per group per thread (fast layout)
  int32_t BPB;      // bits per backpointer field
  int32_t natural;  // 1: slot == edge (K = 8)
  int32_t row_bytes;
};

EXL3_HD inline int32_t bits_per_backpointer(int K) {
  return K == 3 ? 4 : (K >= 5 ? 8 : K);
}

// Thread decomposition of the fast forward kernel for each K (all use 1024
// threads and 64 candidate branches per thread per step):
//   K : G  J  P
//   1 : 16 2  1
//   2 :  4 4  1
//   3 :  4 2  1
//   4 :  4 1  1
//   5 :  2 1  1
//   6 :  2 1  2
//   7 :  2 1  4
// K = 8 has a single group and runs on the generic kernel.
EXL3_HD inline int fast_G(int K) { return K == 1 ? 16 : (K <= 4 ? 4 : 2); }
EXL3_HD inline int fast_J(int K) { return K == 1 ? 2 : (K == 2 ? 4 : (K == 3 ? 2 : 1)); }
EXL3_HD inline int fast_P(int K) { return K == 6 ? 2 : (K == 7 ? 4 : 1); }
EXL3_HD inline bool has_fast_kernel(int K) { return K >= 1 && K <= 7; }

// Backpointer layout of bitrate K. It depends on K only: the generic kernel
// writes the same layout as the fast kernel, so the split forward/backward
// passes may mix kernel variants. K = 8 (no fast kernel) uses one byte per
// edge in edge order.
EXL3_HD inline BpLayout make_layout(int K) {
  BpLayout l;
  l.K = K;
  const int E = 65536 >> K;
  if (!has_fast_kernel(K)) {
    l.G = 1;
    l.J = 1;
    l.BPB = 8;
    l.natural = 1;
  } else {
    l.G = fast_G(K);
    l.J = fast_J(K);
    l.BPB = bits_per_backpointer(K);
    l.natural = 0;
  }
  l.row_bytes = E * l.BPB / 8;
  return l;
}

// Slot of edge e inside a backpointer row.
EXL3_HD inline uint32_t bp_slot(const BpLayout& l, uint32_t e) {
  if (l.natural) return e;
  const uint32_t h = e >> l.K;
  const uint32_t j = e & ((1u << l.K) - 1u);
  const uint32_t G = (uint32_t)l.G, J = (uint32_t)l.J;
  const uint32_t NJ = (1u << l.K) / J;
  const uint32_t unit = (h / G) * NJ + j / J;
  const uint32_t g = h % G;
  const uint32_t local = ((g >> 1) * J + (j % J)) * 2u + (g & 1u);
  return unit * (G * J) + local;
}

EXL3_HD inline uint64_t tile_scratch_bytes(const BpLayout& l, int L) {
  return (uint64_t)(L + 1) * (uint64_t)l.row_bytes;
}

}  // namespace exl3
