/*
 * ORACLE -- test infrastructure only (see oracle/qlora_ref.py header).
 *
 * Bit-level C restatement of the reference's codecs, written with methods
 * deliberately different from both torch and the HIP kernels, so agreement
 * pins them:
 *   - NF4 index: brute-force argmin over the 16 fp32 distances, first
 *     minimum wins (quant_ops.py:114-115);
 *   - bf16 / fp16 / fp8-e4m3fnuz rounding: nearest representable candidate
 *     found by search, exact distances compared in double, ties to the
 *     candidate with an even significand (round-to-nearest-even by its
 *     definition); e4m3fnuz values that round past 240 become NaN (0x80);
 *   - the NF4 table from the decimal literals of quant_ops.py:10-15 (C casts
 *     double -> float with round-to-nearest-even).
 * Build with -O2 -ffp-contract=off (x86-64 SSE arithmetic is IEEE binary32).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define DT_F32 0
#define DT_BF16 1
#define DT_F16 2

static const double kNF4Decimal[16] = {
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0};

static float T[16];
static int t_init = 0;
static void init_table(void) {
  if (t_init) return;
  for (int i = 0; i < 16; ++i) T[i] = (float)kNF4Decimal[i];
  t_init = 1;
}

static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

void ref_nf4_table(float* out) { init_table(); for (int i = 0; i < 16; ++i) out[i] = T[i]; }

/* quant_ops.py:114-115 -- torch.argmin over |n - T_i|; all-NaN row -> 0 */
int ref_nf4_argmin(float n) {
  init_table();
  if (n != n) return 0;
  int best = 0;
  float bd = fabsf(n - T[0]);
  for (int i = 1; i < 16; ++i) {
    float d = fabsf(n - T[i]);
    if (d < bd) { bd = d; best = i; }
  }
  return best;
}

/* ---------------- rounding by nearest-candidate search ---------------- */
/* pick between lo < hi (both representable) for exact value x; ties -> even */
static double pick(double x, double lo, double hi, int lo_even) {
  double dl = x - lo, dh = hi - x;
  if (dl < dh) return lo;
  if (dh < dl) return hi;
  return lo_even ? lo : hi;
}

float ref_round_bf16(float f) {
  if (f != f) return f;
  uint32_t u = f_bits(f);
  uint32_t a = u & 0x7FFFFFFFu, s = u & 0x80000000u;
  if (a >= 0x7F800000u) return f;
  uint32_t lo_b = a & 0xFFFF0000u;
  double x = (double)bits_f(a);
  double lo = (double)bits_f(lo_b);
  if (x == lo) return f;
  uint32_t hi_b = lo_b + 0x10000u;
  double hi = (hi_b >= 0x7F800000u) ? INFINITY : (double)bits_f(hi_b);
  /* values past the largest finite bf16 midpoint round to inf */
  double r = pick(x, lo, hi, ((lo_b >> 16) & 1u) == 0);
  float rf = (float)r;
  return s ? -rf : rf;
}

float ref_round_f16(float f) {
  if (f != f) return f;
  double x = fabs((double)f);
  if (x == 0.0 || isinf(x)) return f;
  int e;
  frexp(x, &e);               /* x = m * 2^e, m in [0.5, 1) */
  int exp2 = e - 1;           /* x in [2^exp2, 2^(exp2+1)) */
  if (exp2 < -14) exp2 = -14; /* subnormal range: fixed quantum 2^-24 */
  double q = ldexp(1.0, exp2 - 10);
  double k = floor(x / q);
  double lo = k * q, hi = (k + 1) * q;
  double r = pick(x, lo, hi, fmod(k, 2.0) == 0.0);
  if (r >= 65520.0 || r > 65504.0) r = INFINITY;
  if (x >= 65520.0) r = INFINITY;
  return (float)(f < 0 ? -r : r);
}

static float ref_round_to(float v, int dt) {
  if (dt == DT_BF16) return ref_round_bf16(v);
  if (dt == DT_F16) return ref_round_f16(v);
  return v;
}

/* e4m3fnuz: value of a code from the format definition */
float ref_fnuz_to_f32(uint8_t c) {
  if (c == 0x80) return NAN;
  int e = (c >> 3) & 15, m = c & 7;
  double v = e == 0 ? ldexp((double)m, -10) : ldexp(8.0 + m, e - 11);
  return (float)((c & 0x80) ? -v : v);
}

/* nearest e4m3fnuz code by search over all magnitudes plus the overflow
 * candidate 256 (mantissa 0, "even"); ties to even mantissa; 256 -> NaN */
uint8_t ref_fnuz_from_f32(float f) {
  if (f != f) return 0x80;
  double x = fabs((double)f);
  if (x >= 256.0) return 0x80;            /* past the overflow candidate */
  int best = -1;
  double bd = INFINITY;
  for (int c = 0; c <= 0x80; ++c) {      /* 0x80 here stands for +256 */
    double v = c == 0x80 ? 256.0 : (double)ref_fnuz_to_f32((uint8_t)c);
    double d = fabs(x - v);
    if (d < bd || (d == bd && (c & 1) == 0 && (best & 1) == 1)) { bd = d; best = c; }
  }
  if (best == 0x80) return 0x80;
  if (best == 0) return 0;
  return (uint8_t)(best | (f < 0 ? 0x80 : 0));
}

/* ------------------------------- codecs ------------------------------- */
static float ld(const void* p, int64_t i, int dt) {
  if (dt == DT_F32) return ((const float*)p)[i];
  uint16_t h = ((const uint16_t*)p)[i];
  if (dt == DT_BF16) return bits_f((uint32_t)h << 16);
  /* fp16 -> fp32 from the definition */
  int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  double v;
  if (e == 0) v = ldexp((double)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexp(1024.0 + m, e - 25);
  return (float)(s ? -v : v);
}

static uint16_t f16_bits_of(float v) {
  /* v is already an fp16 value: encode it */
  uint32_t s = f_bits(v) >> 31;
  double x = fabs((double)v);
  if (v != v) return 0x7E00;
  if (isinf(x)) return (uint16_t)((s << 15) | 0x7C00);
  if (x == 0) return (uint16_t)(s << 15);
  int e;
  frexp(x, &e);
  int exp2 = e - 1;
  if (exp2 < -14) return (uint16_t)((s << 15) | (uint32_t)ldexp(x, 24));
  uint32_t m = (uint32_t)(ldexp(x, 10 - exp2) - 1024.0);
  return (uint16_t)((s << 15) | ((uint32_t)(exp2 + 15) << 10) | m);
}

static void st(void* p, int64_t i, int dt, float v) {
  if (dt == DT_F32) ((float*)p)[i] = v;
  else if (dt == DT_BF16) ((uint16_t*)p)[i] = (uint16_t)(f_bits(ref_round_bf16(v)) >> 16);
  else ((uint16_t*)p)[i] = f16_bits_of(ref_round_f16(v));
}

static float nanmax_abs(float m, float v) {
  float a = fabsf(v);
  if (m != m) return m;
  if (a != a) return a;
  return a > m ? a : m;
}

static float clamp_lo(int dt) {
  /* torch.clamp(min=1e-12) casts the bound to the tensor dtype */
  return ref_round_to((float)1e-12, dt);
}

static float clamp_min(float s, int dt) {
  if (s != s) return s;
  float lo = clamp_lo(dt);
  return s < lo ? lo : s;
}

/* quantize_int4, quant_ops.py:80-126 */
void ref_nf4_quantize(const void* w, int dt, int64_t numel, int64_t bs, uint8_t* packed, void* absmax) {
  int64_t nb = (numel + bs - 1) / bs;
  for (int64_t b = 0; b < nb; ++b) {
    float m = 0.0f;
    for (int64_t i = 0; i < bs; ++i) {
      int64_t e = b * bs + i;
      m = nanmax_abs(m, e < numel ? ld(w, e, dt) : 0.0f);
    }
    float s = clamp_min(m, dt);
    st(absmax, b, dt, s);
    for (int64_t i = 0; i < bs; i += 2) {
      int64_t e = b * bs + i;
      float x0 = e < numel ? ld(w, e, dt) : 0.0f;
      float x1 = e + 1 < numel ? ld(w, e + 1, dt) : 0.0f;
      int i0 = ref_nf4_argmin(ref_round_to(x0 / s, dt));
      int i1 = ref_nf4_argmin(ref_round_to(x1 / s, dt));
      packed[e >> 1] = (uint8_t)(i0 | (i1 << 4));
    }
  }
}

/* dequantize_int4 + `.to(out_dt)`: quant_ops.py:128-150 */
void ref_nf4_dequantize(const uint8_t* packed, const void* absmax, int sdt, int64_t n_packed,
                        int64_t bs, void* out, int odt, int64_t n_out) {
  init_table();
  for (int64_t i = 0; i < n_out && i < 2 * n_packed; ++i) {
    uint8_t byte = packed[i >> 1];
    int c = (i & 1) ? (byte >> 4) : (byte & 15);
    st(out, i, odt, T[c] * ld(absmax, i / bs, sdt));
  }
}

/* double_quantize second stage, double_quant.py:58-87 */
void ref_dq_quantize(const void* c1, int dt, int64_t n, int64_t bs2, int fmt_int8, uint8_t* c2, void* c2s) {
  int64_t nb = (n + bs2 - 1) / bs2;
  for (int64_t b = 0; b < nb; ++b) {
    float m = 0.0f;
    for (int64_t i = 0; i < bs2; ++i) {
      int64_t e = b * bs2 + i;
      m = nanmax_abs(m, e < n ? ld(c1, e, dt) : 0.0f);
    }
    float s = clamp_min(m, dt);
    st(c2s, b, dt, s);
    for (int64_t i = 0; i < bs2; ++i) {
      int64_t e = b * bs2 + i;
      float x = e < n ? ld(c1, e, dt) : 0.0f;
      float nrm = ref_round_to(x / s, dt);
      if (!fmt_int8) {
        c2[e] = ref_fnuz_from_f32(nrm);
      } else {
        float r = nearbyintf(ref_round_to(nrm * 127.0f, dt));
        c2[e] = (uint8_t)(int8_t)(int32_t)r;
      }
    }
  }
}

/* double_dequantize, double_quant.py:99-122 */
void ref_dq_dequantize(const uint8_t* packed, const uint8_t* c2, int fmt_int8, const void* c2s, int sdt,
                       int64_t n_packed, int64_t bs1, int64_t bs2, void* out, int odt, int64_t n_out) {
  init_table();
  for (int64_t i = 0; i < n_out && i < 2 * n_packed; ++i) {
    int64_t b = i / bs1;
    float hi = ld(c2s, b / bs2, sdt);
    float lo = fmt_int8 ? (float)(int8_t)c2[b] / 127.0f : ref_fnuz_to_f32(c2[b]);
    float c1 = lo * hi;
    uint8_t byte = packed[i >> 1];
    int c = (i & 1) ? (byte >> 4) : (byte & 15);
    st(out, i, odt, T[c] * c1);
  }
}

/* quantize_int8, quant_ops.py:17-53; block_size 0 = per row of `cols` */
void ref_int8_quantize(const void* w, int dt, int64_t rows, int64_t cols, int64_t bs, int8_t* q, void* scales) {
  int64_t numel = rows * cols;
  int64_t seg = bs > 0 ? bs : cols;
  int64_t nseg = bs > 0 ? (numel + bs - 1) / bs : rows;
  for (int64_t b = 0; b < nseg; ++b) {
    float m = 0.0f;
    for (int64_t i = 0; i < seg; ++i) {
      int64_t e = b * seg + i;
      m = nanmax_abs(m, e < numel ? ld(w, e, dt) : 0.0f);
    }
    float s = clamp_min(ref_round_to(m / 127.0f, dt), dt);
    st(scales, b, dt, s);
    for (int64_t i = 0; i < seg; ++i) {
      int64_t e = b * seg + i;
      float x = e < numel ? ld(w, e, dt) : 0.0f;
      q[e] = (int8_t)(int32_t)nearbyintf(ref_round_to(x / s, dt));
    }
  }
}

/* the fnuz cast of the FP8 recipe on an array (fp8_linear.py:38,42) */
void ref_fnuz_encode(const float* x, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = ref_fnuz_from_f32(x[i]);
}

void ref_round_array(const float* x, int64_t n, int dt, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = ref_round_to(x[i], dt);
}

/* ------------------------------------------------------------------------
 * Exhaustive check of the kernels' NF4 decision function (64-cell table +
 * one compare, csrc/nf4_tables.h) against the brute-force argmin, over every
 * fp32 value in [-1, 1] (both signs).  Returns the number of mismatches; the
 * first one is written to *first_bad.
 * ------------------------------------------------------------------------ */
int64_t ref_nf4_exhaustive(const uint32_t* cell_thr, const uint8_t* cell_base, int part, int nparts,
                           uint32_t* first_bad) {
  init_table();
  const uint64_t npos = 0x3F800001ull; /* 0x00000000 .. 0x3F800000 */
  const uint64_t total = 2 * npos;
  uint64_t lo = total * (uint64_t)part / (uint64_t)nparts;
  uint64_t hi = total * (uint64_t)(part + 1) / (uint64_t)nparts;
  int64_t bad = 0;
  for (uint64_t k = lo; k < hi; ++k) {
    uint32_t u = k < npos ? (uint32_t)k : (0x80000000u | (uint32_t)(k - npos));
    float n = bits_f(u);
    float c = (n + 1.0f) * 32.0f;
    c = fminf(fmaxf(c, 0.0f), 63.0f);
    int g = (int)c;
    int idx = cell_base[g] + (n > bits_f(cell_thr[g]) ? 1 : 0);
    if (idx != ref_nf4_argmin(n)) {
      if (bad == 0 && first_bad) *first_bad = u;
      ++bad;
    }
  }
  return bad;
}
