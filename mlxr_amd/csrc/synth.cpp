// Deterministic synthetic GGUF weights and activations (host), with the distributions
// of the benchmark configurations.  Used by bench.py and the tests to build inputs; it
// computes nothing that is checked.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../include/mlxr_qgemm.h"

namespace {

struct SplitMix64 {
  uint64_t s;
  explicit SplitMix64(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }  // [0, 1)
  bool have = false;
  double spare = 0.0;
  double normal() {
    if (have) {
      have = false;
      return spare;
    }
    double u1;
    do u1 = uniform(); while (u1 <= 0.0);
    const double u2 = uniform();
    const double r = sqrt(-2.0 * log(u1));
    spare = r * sin(6.283185307179586 * u2);
    have = true;
    return r * cos(6.283185307179586 * u2);
  }
  // uniform integer in [0, n)
  uint32_t below(uint32_t n) { return (uint32_t)(((next() >> 32) * (uint64_t)n) >> 32); }
};

uint16_t f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

// fp32 -> fp16, round to nearest even (values here are finite and far below 65504).
uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    float a;
    memcpy(&a, &ax, 4);
    const double q = (double)a * 16777216.0;
    const double fl = floor(q);
    uint32_t r = (uint32_t)fl;
    const double rem = q - fl;
    if (rem > 0.5 || (rem == 0.5 && (r & 1u))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  const uint32_t rest = ax & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

void put16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}

void fill_bytes(SplitMix64& g, uint8_t* p, int n) {
  for (int i = 0; i < n; i += 8) {
    uint64_t v = g.next();
    for (int j = 0; j < 8 && i + j < n; ++j) p[i + j] = (uint8_t)(v >> (8 * j));
  }
}

}  // namespace

extern "C" {

int mlxr_synth_gguf(int qtype, int N, int K, uint64_t seed, void* out_host) {
  size_t bytes = 0;
  int rc = mlxr_qgemm_gguf_size(qtype, N, K, &bytes);
  if (rc) return rc;
  if (!out_host) return MLXR_E_INVALID;
  if (qtype != MLXR_Q8_0 && qtype != MLXR_Q4_K && qtype != MLXR_Q6_K && qtype != MLXR_Q4_0 && qtype != MLXR_Q4_1 &&
      qtype != MLXR_Q5_K)
    return MLXR_E_UNSUPPORTED;
  const int g = mlxr_qgemm_group_size(qtype);
  if (K % g) return MLXR_E_SHAPE;
  SplitMix64 r(seed);
  uint8_t* p = (uint8_t*)out_host;
  const size_t nblocks = (size_t)N * (size_t)(K / g);
  for (size_t b = 0; b < nblocks; ++b) {
    if (qtype == MLXR_Q8_0) {
      put16(p, f32_to_f16((float)(fabs(r.normal()) * 0.02 / 127.0)));
      for (int i = 0; i < 32; ++i) p[2 + i] = (uint8_t)(int8_t)((int)r.below(255) - 127);
      p += 34;
    } else if (qtype == MLXR_Q4_0) {
      put16(p, f32_to_f16((float)(fabs(r.normal()) * 2e-3)));
      fill_bytes(r, p + 2, 16);
      p += 18;
    } else if (qtype == MLXR_Q4_1) {
      put16(p, f32_to_f16((float)(fabs(r.normal()) * 2e-3)));
      put16(p + 2, f32_to_f16((float)(r.normal() * 8e-3)));
      fill_bytes(r, p + 4, 16);
      p += 20;
    } else if (qtype == MLXR_Q5_K) {
      put16(p, f32_to_f16((float)(fabs(r.normal()) * 1e-3)));
      put16(p + 2, f32_to_f16((float)(fabs(r.normal()) * 1e-3)));
      fill_bytes(r, p + 4, 12);   // scales
      fill_bytes(r, p + 16, 32);  // qh
      fill_bytes(r, p + 48, 128); // qs
      p += 176;
    } else if (qtype == MLXR_Q4_K) {
      put16(p, f32_to_f16((float)(fabs(r.normal()) * 1e-3)));
      put16(p + 2, f32_to_f16((float)(fabs(r.normal()) * 1e-3)));
      fill_bytes(r, p + 4, 12);
      fill_bytes(r, p + 16, 128);
      p += 144;
    } else {
      fill_bytes(r, p, 128);                                                     // ql
      fill_bytes(r, p + 128, 64);                                                // qh
      for (int i = 0; i < 16; ++i) p[192 + i] = (uint8_t)(int8_t)((int)r.below(64) - 32);  // scales
      put16(p + 208, f32_to_f16((float)(fabs(r.normal()) * 1e-3)));             // d
      p += 210;
    }
  }
  return MLXR_OK;
}

int mlxr_synth_act(size_t count, int dtype, uint64_t seed, void* out_host) {
  if (!out_host) return MLXR_E_INVALID;
  SplitMix64 r(seed);
  for (size_t i = 0; i < count; ++i) {
    const float v = (float)r.normal();
    if (dtype == MLXR_BF16) ((uint16_t*)out_host)[i] = f32_to_bf16(v);
    else if (dtype == MLXR_F16) ((uint16_t*)out_host)[i] = f32_to_f16(v);
    else if (dtype == MLXR_F32) ((float*)out_host)[i] = v;
    else return MLXR_E_INVALID;
  }
  return MLXR_OK;
}

}  // extern "C"
