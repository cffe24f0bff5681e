/*
 * exl3_encoder.h — C-ABI of the MI355X (gfx950) EXL3 trellis tile encoder.
 *
 * Drop-in boundary for the reference's native extension `quantize_xpu_ext`
 * (csrc/quantize_xpu/quantize_xpu.cpp:302-357 of
 * alpha2beta/EXL3_Intel_Arc_quantizer). Each entry point below names the
 * reference function it replaces. Conventions, as in the reference:
 *
 *   - every buffer is device memory owned by the caller; nothing is
 *     allocated by these calls;
 *   - work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and runs asynchronously; the caller synchronises;
 *   - the return value is 0 on success, non-zero on a rejected argument or a
 *     launch failure, and exl3_last_error() then describes the problem
 *     (the reference raises RuntimeError from TORCH_CHECK,
 *     quantize_xpu.cpp:73-101,140-157);
 *   - codebook selector cb: 0 = 3INST, 1 = MCG, 2 = MUL1
 *     (quantize_xpu.cpp:85-91); K in 1..8; tile length L in {256, 160},
 *     L = 160 only with MUL1 (quantize_xpu.cpp:93-101).
 *
 * Scratch ("temp_costs" / "temp_edges" in the reference) has a new layout:
 *   temp_costs : fp16 [B][2][E]           terminal path costs of pass 1 / 2,
 *                                          E = 65536 >> K (same as reference)
 *   temp_edges : bytes [B][ROWS][ROWB]    per tile, the fp16 path costs
 *                                          after every S-th step
 *                                          (S = 8, 5, 3, 2, 1, 1, 1, 1 for
 *                                          K = 1..8; ROWB = 2E, group-major),
 *                                          then the header (the L inputs and
 *                                          three int32 fields).
 * where B is the number of tiles the scratch holds (the reference's batch
 * capacity). exl3_scratch_row_bytes() gives ROWB and
 * exl3_scratch_edges_bytes(K, L, 1) / ROWB gives ROWS ((L - 2) / S + 1
 * stored rows plus one header row, two at K = 8 where ROWB = 512). The
 * traceback recomputes the branch of the
 * path at each step from the stored costs. The reference layout stored int16
 * predecessor edges, [B][L][E] (quantize_xpu.cpp:153-157).
 */
#ifndef EXL3_ENCODER_H
#define EXL3_ENCODER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Description of the last failure on the calling thread ("" if none). */
const char* exl3_last_error(void);

/* Library version string. */
const char* exl3_version(void);

/* Default traceback kernel for later calls in this process that do not
 * choose one per call (no counterpart in the reference, whose traceback has
 * one form): 0 = by batch size (default), 1 = per-row tree loads, 2 = whole
 * rows streamed through LDS. Both kernels give identical results. The
 * default is an atomic; exl3_quantize_tiles_tb chooses per call instead.
 * Returns the previous policy, or -1 for a value outside 0..2. */
int exl3_set_traceback_policy(int policy);

/* Replaces decode_codebook (quantize_xpu.cpp:105-110,
 * quantize_kernels.sycl:594-601): fp16 bits of all 65536 states. */
int exl3_decode_codebook(int cb, uint16_t* lut, void* stream);

/* Bytes of one scratch row (ROWB) for bitrate K. The layout depends on K
 * only, so both kernel variants (and the split passes) share it. */
int64_t exl3_scratch_row_bytes(int K);

/* Bytes of temp_edges for `tiles` tiles (replaces the edges term of
 * ScratchEstimator.estimate_scratch, scratch_estimator.py:77-112). */
int64_t exl3_scratch_edges_bytes(int K, int L, int64_t tiles);

/* Position of `edge` inside a stored cost row: (h << K) | k for
 * edge = (k << (16 - 2K)) | h, with part of the digit before at K = 2..5
 * (exposed for host-side checks). */
int64_t exl3_cost_row_slot(int K, int64_t edge);

/* Replaces quantize_tiles (quantize_xpu.cpp:112-167,
 * quantize_kernels.sycl:603-656): full two-pass tail-biting encode of n
 * tiles. in: f32 [n][L] in kernel order holding fp16-representable values;
 * out_w: f32 [n][L] reconstruction (kernel order); out_idx: int16 [n][L]
 * 16-bit states. temp_costs/temp_edges hold batch_cap tiles; tiles are
 * processed in chunks of min(batch_cap, wave_cap) (wave_cap <= 0: no cap).
 * generic = 1 selects the reference-structured kernel. */
int exl3_quantize_tiles(const float* in, float* out_w, int16_t* out_idx, uint16_t* temp_costs,
                        uint8_t* temp_edges, int64_t batch_cap, int64_t n, int K, int cb, int L,
                        int generic, int64_t wave_cap, void* stream);

/* exl3_quantize_tiles with the traceback kernel chosen for this call only
 * (no counterpart in the reference, whose traceback has one form):
 * traceback = 0 by batch size, 1 per-row tree loads, 2 whole rows streamed
 * through LDS, -1 the process default of exl3_set_traceback_policy. Results
 * are identical for every choice; the process default is not changed, so
 * callers on several threads or streams may choose differently. */
int exl3_quantize_tiles_tb(const float* in, float* out_w, int16_t* out_idx,
                           uint16_t* temp_costs, uint8_t* temp_edges, int64_t batch_cap,
                           int64_t n, int K, int cb, int L, int generic, int64_t wave_cap,
                           int traceback, void* stream);

/* Bytes of the library's static scratch for exl3_quantize_tiles_noalloc. */
#define EXL3_NOALLOC_SCRATCH_BYTES ((int64_t)512 << 20)

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): exl3_quantize_tiles for n tiles with its temp_costs and
 * temp_edges in a static device array of EXL3_NOALLOC_SCRATCH_BYTES (512
 * MiB) that each GPU holds from library load until the process ends. No
 * hipMalloc, hipFree or allocating library call is made. Limit: all n tiles
 * must fit at once, n <= floor((EXL3_NOALLOC_SCRATCH_BYTES - 255) /
 * (4 (65536 >> K) + exl3_scratch_edges_bytes(K, L, 1))), e.g. 303 tiles at
 * K = 2 and 500 at K = 4 (L = 256); larger n is rejected with an error and
 * nothing is launched. Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (on different streams, or from several threads
 * without ordering) race and corrupt each other's results. Results equal
 * exl3_quantize_tiles'. in / out_w / out_idx as there; the device is the
 * one current on the calling thread, which must be `stream`'s. */
int exl3_quantize_tiles_noalloc(const float* in, float* out_w, int16_t* out_idx, int64_t n,
                                int K, int cb, int L, int generic, void* stream);

/* Replaces quantize_tiles_forward_pass (quantize_xpu.cpp:169-215,
 * quantize_kernels.sycl:658-704): one forward add-compare-select pass over
 * the ring with rotation `roll`; tile t is constrained to start from edge
 * pre_states[t] when that is >= 0. Writes every stored cost row, the tile
 * header and the terminal costs to
 * temp_costs[t][cost_slot]. n <= batch capacity. generic = 1 selects the
 * reference-structured kernel. */
int exl3_forward_pass(const float* in, uint16_t* temp_costs, uint8_t* temp_edges,
                      const int32_t* pre_states, int64_t n, int K, int cb, int L, int roll,
                      int cost_slot, int generic, void* stream);

/* Replaces quantize_tiles_backward_pass (quantize_xpu.cpp:217-259,
 * quantize_kernels.sycl:706-736). write = 0: end_states[t] = edge reached
 * at ring row 0 walking back from the argmin of temp_costs[t][cost_slot];
 * write = 1: walk back from end_states[t] writing out_w / out_idx. */
int exl3_backward_pass(const uint16_t* temp_costs, const uint8_t* temp_edges, float* out_w,
                       int16_t* out_idx, int32_t* end_states, int64_t n, int K, int cb, int L,
                       int roll, int cost_slot, int write, void* stream);

/* Host-side preparation of the reference wrapper (xpu_quantizer.py:649-655)
 * on the device: out[t][i] = fp16-rounded raw[t][perm[i]] (permute = 1,
 * tensor-core permutation, L = 256) or raw[t][i] (permute = 0), as f32.
 * nan_count (device int32, may be NULL) is incremented once per NaN input
 * value; the reference's NaN behaviour is not reproduced, callers reject
 * batches with a non-zero count. */
int exl3_prepare_tiles(const float* raw, float* out, int64_t n, int L, int permute,
                       int32_t* nan_count, void* stream);

/* Host-side post-processing of the reference wrapper
 * (xpu_quantizer.py:926-976) on the device, per tile:
 *   packed[t][16K]   pack_trellis + swap16_storage (L = 256 only; may be NULL)
 *   path_cost[t]     sequential fp16 cost along the chosen path
 *   distortion[t]    float32 sum((orig - recon)^2) in numpy's pairwise order
 *   recon_orig[t][L] fp16 reconstruction in original order
 * x: kernel-order f32 inputs (fp16 values); raw: original-order f32 tiles
 * (used for the distortion when permuted = 1, else may be NULL). */
int exl3_finalize_tiles(const float* x, const float* raw, const float* out_w,
                        const int16_t* out_idx, uint16_t* packed, float* path_cost,
                        float* distortion, uint16_t* recon_orig, int64_t n, int K, int L,
                        int permuted, void* stream);

/* pack_trellis + swap16_storage (trellis_format.py:120-174) for n tiles of
 * 256 int16 states: packed is uint16 [n][16K]. */
int exl3_pack_trellis(const int16_t* states, uint16_t* packed, int64_t n, int K, void* stream);

/* decode_states (trellis_format.py:181-213) for n packed tiles, the read-back
 * of unpack_module_trellis (serialization.py:65-84): states[t][i] is the
 * 16-bit window of tile t's bitstream ending at bit (i + 1) K, circular. */
int exl3_unpack_trellis(const uint16_t* packed, int16_t* states, int64_t n, int K, void* stream);

/* fp16 fused multiply-add probe (xpu_probe.py:153-272): out[i] =
 * fp16(a[i]*a[i] + c[i]) with one rounding (mode 0) or the two-rounding
 * expression fp16(fp16(a*a) + c) (mode 1). */
int exl3_probe_hfma(const uint16_t* a, const uint16_t* c, uint16_t* out, int64_t n, int mode,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_ENCODER_H */
