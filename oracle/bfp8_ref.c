/* bfloat8_b codec restated in plain C - TEST ORACLE ONLY.
 *
 * The reference fixes only the tile size (32*32 + 64 = 1088 bytes,
 * python/ttl/dtype_utils.py:174-175).  Format checked here (the MI355X
 * library implements the same contract independently):
 *   tile = 64 exponent bytes + 1024 element bytes, faces (0-15,0-15),
 *   (0-15,16-31), (16-31,0-15), (16-31,16-31); exponent 16*f + r; element
 *   byte 64 + 256*f + 16*r + c = sign(bit 7) | magnitude m (bits 6..0);
 *   value = (-1)^s * m * 2^(e-133) (+-inf when that exceeds the bf16 range,
 *   possible only for e = 255, which packing finite data never emits); pack: e = max biased exponent of the 16
 *   values of a face row, m = round-half-even(|x| 2^(133-e)) capped at 127.
 * Written with integer arithmetic only (no libm), so it shares no code path
 * with the library's double / ldexp implementation.
 */
#include <stdint.h>
#include <string.h>

static int face_of(int r, int c) { return ((r >> 4) << 1) | (c >> 4); }

/* |x| * 2^(133 - e) rounded half-to-even, computed on the fp32 bit pattern */
static uint32_t quantise(uint32_t bits, int e) {
  uint32_t ex = (bits >> 23) & 0xff, frac = bits & 0x7fffff;
  uint64_t sig;   /* integer significand */
  int shift;      /* value = sig * 2^(shift) * 2^(133-e) */
  if (ex == 0) { sig = frac; shift = -149; }          /* subnormal / zero */
  else { sig = frac | 0x800000u; shift = (int)ex - 150; }
  int s = shift + 133 - e;                            /* m = sig * 2^s */
  if (sig == 0) return 0;
  if (s >= 0) { uint64_t m = sig << (s > 40 ? 40 : s); return m > 127 ? 127 : (uint32_t)m; }
  int r = -s;
  if (r > 63) return 0;
  uint64_t q = sig >> r, rem = sig & ((1ull << r) - 1), half = 1ull << (r - 1);
  if (rem > half || (rem == half && (q & 1))) q += 1;
  return q > 127 ? 127 : (uint32_t)q;
}

void oracle_bfp8_pack(const float* src, uint8_t* dst, int64_t rows, int64_t cols) {
  int64_t ntc = cols / 32;
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < ntc; ++tc) {
      uint8_t* t = dst + (tr * ntc + tc) * 1088;
      for (int r = 0; r < 32; ++r)
        for (int h = 0; h < 2; ++h) {
          uint32_t bits[16];
          int e = 0;
          for (int c = 0; c < 16; ++c) {
            memcpy(&bits[c], &src[(tr * 32 + r) * cols + tc * 32 + h * 16 + c], 4);
            int ex = (bits[c] >> 23) & 0xff;
            if (ex > e) e = ex;
          }
          int f = face_of(r, h * 16);
          t[16 * f + (r & 15)] = (uint8_t)e;
          for (int c = 0; c < 16; ++c)
            t[64 + 256 * f + 16 * (r & 15) + c] =
                (uint8_t)(((bits[c] >> 31) << 7) | quantise(bits[c] & 0x7fffffffu, e));
        }
    }
}

/* exact bf16 of (-1)^s m 2^(e-133), built from integer fields */
uint16_t oracle_bfp8_decode(uint8_t e, uint8_t b) {
  uint32_t s = b >> 7, m = b & 0x7f;
  if (m == 0) return (uint16_t)(s << 15);
  int p = 6;
  while (!(m & (1u << p))) --p;          /* leading one */
  int E = p + (int)e - 6;                /* biased bf16 exponent of m 2^(e-133) */
  uint32_t out;
  if (E >= 255) out = 0x7f80;  /* e = 255 (never packed from finite data): overflow -> inf */
  else if (E >= 1) out = ((uint32_t)E << 7) | ((m << (7 - p)) & 0x7f);  /* normal */
  else out = m << e;  /* subnormal: field = value / 2^-133 = m 2^e (< 128 here) */
  return (uint16_t)((s << 15) | out);
}

void oracle_bfp8_unpack(const uint8_t* src, uint16_t* dst, int64_t rows, int64_t cols) {
  int64_t ntc = cols / 32;
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < ntc; ++tc) {
      const uint8_t* t = src + (tr * ntc + tc) * 1088;
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          int f = face_of(r, c);
          dst[(tr * 32 + r) * cols + tc * 32 + c] =
              oracle_bfp8_decode(t[16 * f + (r & 15)], t[64 + 256 * f + 16 * (r & 15) + (c & 15)]);
        }
    }
}

/* ---------------------------------------------------------------------------
 * bfloat4_b (576-byte tiles, python/ttl/dtype_utils.py:176-177) - TEST ORACLE.
 * Same faces and shared exponents; element nibble = sign (bit 3) | magnitude m
 * (bits 2..0), byte 64 + 128*f + 8*r + c/2 (low nibble: even c);
 * value = (-1)^s m 2^(e-129); pack m = round-half-even(|x| 2^(129-e)) <= 7.
 */

/* |x| * 2^(129 - e) rounded half-to-even, capped at 7 (integer arithmetic) */
static uint32_t quantise4(uint32_t bits, int e) {
  uint32_t ex = (bits >> 23) & 0xff, frac = bits & 0x7fffff;
  uint64_t sig;
  int shift;
  if (ex == 0) { sig = frac; shift = -149; }
  else { sig = frac | 0x800000u; shift = (int)ex - 150; }
  int s = shift + 129 - e;
  if (sig == 0) return 0;
  if (s >= 0) { uint64_t m = sig << (s > 40 ? 40 : s); return m > 7 ? 7 : (uint32_t)m; }
  int r = -s;
  if (r > 63) return 0;
  uint64_t q = sig >> r, rem = sig & ((1ull << r) - 1), half = 1ull << (r - 1);
  if (rem > half || (rem == half && (q & 1))) q += 1;
  return q > 7 ? 7 : (uint32_t)q;
}

void oracle_bfp4_pack(const float* src, uint8_t* dst, int64_t rows, int64_t cols) {
  int64_t ntc = cols / 32;
  memset(dst, 0, (size_t)((rows / 32) * ntc * 576));
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < ntc; ++tc) {
      uint8_t* t = dst + (tr * ntc + tc) * 576;
      for (int r = 0; r < 32; ++r)
        for (int h = 0; h < 2; ++h) {
          uint32_t bits[16];
          int e = 0;
          for (int c = 0; c < 16; ++c) {
            memcpy(&bits[c], &src[(tr * 32 + r) * cols + tc * 32 + h * 16 + c], 4);
            int ex = (bits[c] >> 23) & 0xff;
            if (ex > e) e = ex;
          }
          int f = face_of(r, h * 16);
          t[16 * f + (r & 15)] = (uint8_t)e;
          for (int c = 0; c < 16; ++c) {
            uint32_t nib = ((bits[c] >> 31) << 3) | quantise4(bits[c] & 0x7fffffffu, e);
            t[64 + 128 * f + 8 * (r & 15) + (c >> 1)] |= (uint8_t)(nib << (4 * (c & 1)));
          }
        }
    }
}

/* exact bf16 of (-1)^s m 2^(e-129), built from integer fields */
uint16_t oracle_bfp4_decode(uint8_t e, uint8_t nib) {
  uint32_t s = (nib >> 3) & 1, m = nib & 7;
  if (m == 0) return (uint16_t)(s << 15);
  int p = 2;
  while (!(m & (1u << p))) --p;          /* leading one */
  int E = p + (int)e - 2;                /* biased bf16 exponent of m 2^(e-129) */
  uint32_t out;
  if (E >= 255) out = 0x7f80;            /* e >= 253 with m >= 4: overflow -> inf */
  else if (E >= 1) out = ((uint32_t)E << 7) | ((m << (7 - p)) & 0x7f);
  else out = m << (e + 4);               /* subnormal: field = value / 2^-133 */
  return (uint16_t)((s << 15) | out);
}

void oracle_bfp4_unpack(const uint8_t* src, uint16_t* dst, int64_t rows, int64_t cols) {
  int64_t ntc = cols / 32;
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < ntc; ++tc) {
      const uint8_t* t = src + (tr * ntc + tc) * 576;
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          int f = face_of(r, c);
          uint8_t byte = t[64 + 128 * f + 8 * (r & 15) + ((c & 15) >> 1)];
          dst[(tr * 32 + r) * cols + tc * 32 + c] =
              oracle_bfp4_decode(t[16 * f + (r & 15)], (uint8_t)((byte >> (4 * (c & 1))) & 0xf));
        }
    }
}
