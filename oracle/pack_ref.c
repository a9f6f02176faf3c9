/* Plain-C restatement of the reference's KV storage quantizers and attention -- TEST
 * INFRASTRUCTURE ONLY (used by tests/ as an independent second restatement of oracle/ref.py;
 * never linked into or called by the product library).
 *
 * Reference: stfurkan/bitgpu v0.19.1.
 *   q8 pack   : shaders/copy_kv8.wgsl:24-40 + the WGSL pack4x8snorm definition
 *               code = floor(0.5 + 127 * clamp(v / s, -1, 1)), s = max(max|v|, 1e-30)
 *   q8 dequant: shaders/attention_sg_kv8.wgsl:40 (max(c / 127, -1) * s)
 *   f16 pack  : shaders/copy_kv16.wgsl:13, IEEE binary16 round-to-nearest-even, done here
 *               with integer bit manipulation (independent of any float16 library)
 *   attention : tools/reference.py:158-175 computed in double precision with explicit loops
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; every f32 operation rounds once).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float absf(float x) { return x < 0.0f ? -x : x; }

/* rows x D f32 -> int8 codes (natural element order) + rows x (D/block) f32 scales */
void oracle_q8_pack(const float* x, int rows, int D, int block, int8_t* codes, float* scales) {
  const float tiny = 1e-30f;
  for (int r = 0; r < rows; r++) {
    for (int b = 0; b < D / block; b++) {
      const float* v = x + (size_t)r * D + (size_t)b * block;
      float m = 0.0f;
      for (int i = 0; i < block; i++) {
        float a = absf(v[i]);
        if (a > m) m = a;
      }
      float s = m > tiny ? m : tiny;
      scales[(size_t)r * (D / block) + b] = s;
      for (int i = 0; i < block; i++) {
        volatile float e = v[i] / s;          /* one correctly rounded division */
        float ec = e < -1.0f ? -1.0f : (e > 1.0f ? 1.0f : e);
        volatile float t = 127.0f * ec;       /* rounded product, never fused */
        volatile float u = t + 0.5f;          /* rounded sum */
        codes[(size_t)r * D + (size_t)b * block + i] = (int8_t)floorf(u);
      }
    }
  }
}

void oracle_q8_dequant(const int8_t* codes, const float* scales, int rows, int D, int block, float* out) {
  for (int r = 0; r < rows; r++)
    for (int i = 0; i < D; i++) {
      volatile float u = (float)codes[(size_t)r * D + i] / 127.0f;
      if (u < -1.0f) u = -1.0f;
      out[(size_t)r * D + i] = u * scales[(size_t)r * (D / block) + i / block];
    }
}

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even (subnormals, inf, nan). */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ex = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (ex == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  int32_t e = (int32_t)ex - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000u;             /* implicit bit */
    int shift = 14 - e;                       /* 24-bit significand -> subnormal f16 */
    uint32_t hm = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = man >> 13;
  uint32_t rem = man & 0x1fffu;
  uint32_t out = sign | ((uint32_t)e << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) out++; /* carry into exponent is correct */
  return (uint16_t)out;
}

void oracle_f16_pack(const float* x, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; i++) out[i] = oracle_f32_to_f16(x[i]);
}

/* Brute-force causal GQA attention in double precision over a cache.
 * q: [S,H,D]; k,v: [L,KV,D]; valid: [L] (NULL = all); query s attends j <= pos_base + s.
 * scale <= 0 selects 1/sqrt(D). out: [S,H,D] f32. */
void oracle_attention_f64(const float* q, const float* k, const float* v, const uint8_t* valid, int S, int H,
                          int KV, int D, int L, int pos_base, double scale, float* out) {
  if (scale <= 0.0) scale = 1.0 / sqrt((double)D);
  int rep = H / KV;
  double sc_buf[65536];
  double acc[512];
  for (int s = 0; s < S; s++)
    for (int h = 0; h < H; h++) {
      int kvh = h / rep;
      const float* qr = q + ((size_t)s * H + h) * D;
      int last = pos_base + s;
      double mx = -1e300;
      for (int j = 0; j < L && j < 65536; j++) {
        double d = 0.0;
        const float* kr = k + ((size_t)j * KV + kvh) * D;
        for (int i = 0; i < D; i++) d += (double)qr[i] * (double)kr[i];
        d *= scale;
        int ok = j <= last && (!valid || valid[j]);
        sc_buf[j] = ok ? d : -INFINITY;
        if (ok && d > mx) mx = d;
      }
      double den = 0.0;
      for (int i = 0; i < D; i++) acc[i] = 0.0;
      for (int j = 0; j < L && j < 65536; j++) {
        if (sc_buf[j] == -INFINITY) continue;
        double p = exp(sc_buf[j] - mx);
        den += p;
        const float* vr = v + ((size_t)j * KV + kvh) * D;
        for (int i = 0; i < D; i++) acc[i] += p * (double)vr[i];
      }
      float* o = out + ((size_t)s * H + h) * D;
      for (int i = 0; i < D; i++) o[i] = (float)(acc[i] / den);
    }
}
