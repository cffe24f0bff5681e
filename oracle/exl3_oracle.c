/*
 * C restatement of the EXL3 trellis tile encoder — TEST INFRASTRUCTURE ONLY.
 *
 * Restates exl3_quant/reference_encoder.py (ReferenceTrellisEncoder,
 * reference_encoder.py:99-324) and the format helpers of
 * exl3_quant/trellis_format.py:41-174 of the reference, with the same fp16
 * semantics:
 *
 *   dh  = fp16(val - w)                  fp16 subtract, one rounding
 *   err = fp16(dh*dh)                    step 0 (masked to +inf where
 *                                        pred != pre_state if pre_state >= 0)
 *   err = fp16(dh*dh + cost_prev[pred])  steps 1..L-1, ONE rounding (fused)
 *
 * Every fp16 result is produced by evaluating the operation exactly in
 * double precision and rounding the double directly to fp16 (round to
 * nearest even, subnormals kept). For the sums above the double evaluation
 * is exact whenever the fp16 result is finite (|dh*dh| < 2^16, so the
 * exponent span of the operands stays within 53 bits), hence this is a
 * correctly rounded fused multiply-add. Going double -> float -> half would
 * round twice; the direct conversion below never does.
 *
 * Per edge, branch k = 0 initialises the running minimum and a later branch
 * replaces it only when strictly smaller (fp16 '<', NaN compares false):
 * reference_encoder.py:169-176,193-199. Terminal argmin: lowest index of the
 * minimum; 0 if no cost is finite or all costs are +inf (:206-214).
 *
 * Built by oracle/Makefile into oracle/libexl3_oracle.so; called through
 * ctypes by oracle/c_oracle.py. Used by the tests as the checker and by
 * bench.py as the CPU baseline ("port"); never by the product.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ fp16 */

static double g_h2d[65536];
static int g_h2d_ready = 0;

static double half_bits_to_double(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int exp = (h >> 10) & 0x1F;
  const int man = h & 0x3FF;
  double v;
  if (exp == 0) {
    v = ldexp((double)man, -24);
  } else if (exp == 31) {
    v = man ? NAN : INFINITY;
  } else {
    v = ldexp((double)(man | 0x400), exp - 25);
  }
  return sign ? -v : v;
}

static void init_tables(void) {
  if (g_h2d_ready) return;
  for (int i = 0; i < 65536; ++i) g_h2d[i] = half_bits_to_double((uint16_t)i);
  g_h2d_ready = 1;
}

/* Round a double to the nearest fp16 (ties to even), directly. */
static inline uint16_t double_to_half_bits(double x) {
  uint64_t b;
  memcpy(&b, &x, sizeof b);
  const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  const uint64_t a = b & 0x7FFFFFFFFFFFFFFFull;
  if (a >= 0x7FF0000000000000ull) {                 /* inf / NaN */
    if (a == 0x7FF0000000000000ull) return sign | 0x7C00u;
    return sign | 0x7E00u | (uint16_t)((a >> 42) & 0x1FFu);
  }
  const int e = (int)(a >> 52) - 1023;               /* unbiased exponent */
  if (e >= 16) return sign | 0x7C00u;
  if (e < -26) return sign;                          /* < 2^-26: rounds to 0 */
  const uint64_t m = (a & 0x000FFFFFFFFFFFFFull) | (1ull << 52);
  /* Number of low significand bits dropped: normal results keep 11 bits,
   * subnormal results keep bits down to 2^-24. */
  const int shift = (e >= -14) ? 42 : (28 - e);
  uint64_t q = m >> shift;
  const uint64_t rem = m & ((1ull << shift) - 1);
  const uint64_t halfway = 1ull << (shift - 1);
  if (rem > halfway || (rem == halfway && (q & 1))) ++q;
  if (e >= -14) {
    int he = e + 15;
    if (q == 2048) { q = 1024; ++he; }
    if (he >= 31) return sign | 0x7C00u;
    return sign | (uint16_t)(he << 10) | (uint16_t)(q - 1024);
  }
  return sign | (uint16_t)q;                         /* q == 1024 is the min normal */
}

static inline double h2d(uint16_t h) { return g_h2d[h]; }

/* fp16 '<' on bit patterns via exact doubles (NaN compares false). */
static inline int half_lt(uint16_t a, uint16_t b) { return h2d(a) < h2d(b); }

/* ------------------------------------------------------------- codebook */

/* trellis_format.py:41-81 / codebook.cuh:56-123 */
static uint16_t decode_state(int cb, uint32_t s) {
  if (cb == 2) {
    const uint32_t x = s * 0x83DCD12Du;
    const uint32_t bsum = (x & 0xFFu) + ((x >> 8) & 0xFFu) + ((x >> 16) & 0xFFu) + (x >> 24);
    const double h = h2d((uint16_t)(0x6400u + bsum));
    return double_to_half_bits(h * h2d(0x1EEE) + h2d(0xC931));
  }
  uint32_t x = (cb == 0) ? (s * 89226354u + 64248484u) : (s * 0xCBAC1FEDu);
  x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
  return double_to_half_bits(h2d((uint16_t)(x & 0xFFFFu)) + h2d((uint16_t)(x >> 16)));
}

ORACLE_API void exl3o_codebook_lut(int cb, uint16_t* out) {
  init_tables();
  for (uint32_t s = 0; s < 65536u; ++s) out[s] = decode_state(cb, s);
}

ORACLE_API uint16_t exl3o_half_from_double(double x) { return double_to_half_bits(x); }

ORACLE_API void exl3o_fma_f16(const uint16_t* a, const uint16_t* c, uint16_t* out, int64_t n) {
  init_tables();
  for (int64_t i = 0; i < n; ++i) out[i] = double_to_half_bits(h2d(a[i]) * h2d(a[i]) + h2d(c[i]));
}

/* ------------------------------------------------------------- encoder */

static inline int ring_index(int i, int roll, int L) {
  const int ri = i + roll;
  return ri >= L ? ri - L : ri;
}

/* reference_encoder.py:130-204. Writes the chosen predecessor edge of every
 * edge at ring row ri into edges[ri*E + e]; leaves the terminal costs in
 * cost_out. lut: fp16 bits of every state. */
static void forward_pass(const uint16_t* lut, const uint16_t* tile16, int K, int L, int roll,
                         int pre_state, uint16_t* edges, uint16_t* cost_a, uint16_t* cost_b,
                         uint16_t** cost_out, uint16_t* rows) {
  const int E = 65536 >> K, Kr = 16 - K, Q = 1 << K;
  uint16_t* prev = cost_a;
  uint16_t* next = cost_b;
  for (int i = 0; i < L; ++i) {
    const int ri = ring_index(i, roll, L);
    const double w = h2d(tile16[ri]);
    uint16_t* row = edges + (size_t)ri * E;
    for (int e = 0; e < E; ++e) {
      uint16_t best = 0, best_pred = 0;
      for (int k = 0; k < Q; ++k) {
        const uint32_t sigma = ((uint32_t)k << Kr) | (uint32_t)e;
        const uint16_t pred = (uint16_t)(sigma >> K);
        const double dh = h2d(double_to_half_bits(h2d(lut[sigma]) - w));
        uint16_t err;
        if (i == 0) {
          err = double_to_half_bits(dh * dh);
          if (pre_state >= 0 && (int)pred != pre_state) err = 0x7C00u;
        } else {
          err = double_to_half_bits(dh * dh + h2d(prev[pred]));
        }
        if (k == 0 || half_lt(err, best)) {
          best = err;
          best_pred = pred;
        }
      }
      next[e] = best;
      row[e] = best_pred;
    }
    if (rows) memcpy(rows + (size_t)i * E, next, (size_t)E * sizeof(uint16_t));
    uint16_t* t = prev;
    prev = next;
    next = t;
  }
  *cost_out = prev;
}

static int argmin_cost(const uint16_t* costs, int E) {
  int any_finite = 0, all_inf = 1, best = 0;
  for (int e = 0; e < E; ++e) {
    const double c = h2d(costs[e]);
    if (isfinite(c)) any_finite = 1;
    if (costs[e] != 0x7C00u) all_inf = 0;
  }
  if (!any_finite || all_inf) return 0;
  /* np.argmin: first minimum; a NaN counts as the minimum (first NaN wins). */
  for (int e = 0; e < E; ++e) {
    if (isnan(h2d(costs[e]))) return e;
  }
  for (int e = 1; e < E; ++e) {
    if (h2d(costs[e]) < h2d(costs[best])) best = e;
  }
  return best;
}

/* Per-tile outputs in kernel (ring) order. */
typedef struct {
  uint16_t* idx;       /* L states */
  uint16_t* rec;       /* L fp16 reconstruction, kernel order */
  int32_t* end_state;
  uint16_t* path_cost; /* fp16 bits of c2[end_state] */
  int32_t* best_edge;  /* pass-1 terminal argmin */
} tile_out_t;

static void encode_one(const uint16_t* lut, const uint16_t* tile16, int K, int L, uint16_t* edges,
                       uint16_t* ca, uint16_t* cb_, tile_out_t o) {
  const int E = 65536 >> K;
  uint16_t* c1;
  forward_pass(lut, tile16, K, L, L / 2, -1, edges, ca, cb_, &c1, NULL);
  const int best = argmin_cost(c1, E);
  /* backward(write=False): reference_encoder.py:239-249 */
  int edge = best;
  for (int i = L - 1; i >= 0; --i) {
    const int ri = ring_index(i, L / 2, L);
    edge = edges[(size_t)ri * E + edge];
    if (ri == 0) break;
  }
  const int end_state = edge;
  uint16_t* c2;
  forward_pass(lut, tile16, K, L, 0, end_state, edges, ca, cb_, &c2, NULL);
  edge = end_state;
  for (int i = L - 1; i >= 0; --i) {
    const int prev = edges[(size_t)i * E + edge];
    const uint16_t state = (uint16_t)((prev << K) | edge);
    edge = prev;
    o.idx[i] = state;
    o.rec[i] = lut[state];
  }
  *o.end_state = end_state;
  *o.path_cost = c2[end_state];
  *o.best_edge = best;
}

/* Encode n tiles of fp16 bits (already in kernel order). Returns 0 on
 * success, -1 on bad arguments, -2 on allocation failure. */
ORACLE_API int exl3o_encode_tiles(const uint16_t* tiles16, int64_t n, int K, int cb, int L,
                                  uint16_t* out_idx, uint16_t* out_rec, int32_t* end_states,
                                  uint16_t* path_costs, int32_t* best_edges, int threads) {
  if (K < 1 || K > 8 || cb < 0 || cb > 2 || L <= 0 || (L & 1) || n < 0) return -1;
  init_tables();
  uint16_t* lut = (uint16_t*)malloc(65536 * sizeof(uint16_t));
  if (!lut) return -2;
  exl3o_codebook_lut(cb, lut);
  const int E = 65536 >> K;
  int status = 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
#pragma omp parallel
  {
    uint16_t* edges = (uint16_t*)malloc((size_t)L * E * sizeof(uint16_t));
    uint16_t* ca = (uint16_t*)malloc((size_t)E * sizeof(uint16_t));
    uint16_t* cbuf = (uint16_t*)malloc((size_t)E * sizeof(uint16_t));
    if (!edges || !ca || !cbuf) {
#pragma omp atomic write
      status = -2;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int64_t t = 0; t < n; ++t) {
        tile_out_t o = {out_idx + t * L, out_rec + t * L, end_states + t, path_costs + t,
                        best_edges + t};
        encode_one(lut, tiles16 + t * L, K, L, edges, ca, cbuf, o);
      }
    }
    free(edges);
    free(ca);
    free(cbuf);
  }
  free(lut);
  return status;
}

/* One forward pass on one tile, exposing the full predecessor table
 * (reference_encoder.py:130-204) and, when rows is not NULL, the cost vector
 * after every step (rows[i*E + e]); used to pin forward() on its own. */
ORACLE_API int exl3o_forward_pass(const uint16_t* tile16, int K, int cb, int L, int roll,
                                  int pre_state, uint16_t* edges, uint16_t* costs_out,
                                  uint16_t* rows) {
  if (K < 1 || K > 8 || cb < 0 || cb > 2 || L <= 0 || (L & 1)) return -1;
  init_tables();
  const int E = 65536 >> K;
  uint16_t* lut = (uint16_t*)malloc(65536 * sizeof(uint16_t));
  uint16_t* ca = (uint16_t*)malloc((size_t)E * sizeof(uint16_t));
  uint16_t* cbuf = (uint16_t*)malloc((size_t)E * sizeof(uint16_t));
  if (!lut || !ca || !cbuf) {
    free(lut); free(ca); free(cbuf);
    return -2;
  }
  exl3o_codebook_lut(cb, lut);
  uint16_t* out;
  forward_pass(lut, tile16, K, L, roll, pre_state, edges, ca, cbuf, &out, rows);
  memcpy(costs_out, out, (size_t)E * sizeof(uint16_t));
  free(lut); free(ca); free(cbuf);
  return 0;
}

/* pack_trellis + swap16_storage for n tiles (trellis_format.py:120-174). */
ORACLE_API void exl3o_pack_tiles(const uint16_t* states, int64_t n, int K, uint16_t* out) {
  const int words = 16 * K;
  for (int64_t t = 0; t < n; ++t) {
    const uint16_t* s = states + t * 256;
    uint16_t* o = out + t * words;
    for (int span = 0; span < 16; ++span) {
      uint32_t buf = 0;
      int held = 32, j = span * K;
      for (int i = 0; i < 16; ++i) {
        held -= K;
        buf |= (uint32_t)(s[span * 16 + i] & ((1u << K) - 1u)) << held;
        if (held <= 16) {
          o[j++] = (uint16_t)(buf >> 16);
          buf <<= 16;
          held += 16;
        }
      }
    }
    for (int w = 0; w < words; w += 2) {
      const uint16_t lo = o[w];
      o[w] = o[w + 1];
      o[w + 1] = lo;
    }
  }
}
