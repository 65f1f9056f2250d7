// Shared device helpers for the gfx950 KV-cache kernels: element types, 8-wide vector
// loads/stores with conversion to bf16, fp8 e4m3fn encoding, and the host-side error state.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/solarkv.h"

namespace skv {

typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;  // the only head_dim the kernels are built for
constexpr int kTile = 64;      // keys per attention tile == frame padding granule

inline int padded_tokens(int T) { return (T + kTile - 1) / kTile * kTile; }

// ---- host error state (one message per host thread) ---------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

// ---- host launch helpers (defined in skv_attention.hip) -----------------------------------
int cu_count();  // compute units of the current device (256 on MI355X)
// skv_attention_ex (or, with plan != nullptr, skv_attention_plan) on a copy of `d` whose
// workspace is (ws, ws_bytes); ws == nullptr means none.  Clears and sets the error state.
int attention_with_workspace(const skv_attention_desc* d, void* ws, int64_t ws_bytes,
                             skv_stream_t stream, skv_launch_plan* plan);

// ---- element traits ---------------------------------------------------------------------
// A "vec8" is 8 consecutive elements of one row; all pool and token layouts keep them
// contiguous and 8-element aligned, so they move as 16 B (bf16) or 32 B (fp32).
template <typename T>
struct Vec8;

// Streaming (nontemporal) 16 B accesses for data touched once per launch: the byte movers use
// them so chunk sources, pool writes and gathered frames do not displace cached K/V tiles.
__device__ inline u32x4 ld_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ inline void st_nt(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

template <>
struct Vec8<bf16> {
  u32x4 r;
  __device__ static Vec8 load(const bf16* p) {
    Vec8 v;
    v.r = *reinterpret_cast<const u32x4*>(p);
    return v;
  }
  __device__ void store(bf16* p) const { *reinterpret_cast<u32x4*>(p) = r; }
  __device__ static Vec8 load_nt(const bf16* p) {
    Vec8 v;
    v.r = ld_nt(p);
    return v;
  }
  __device__ void store_nt(bf16* p) const { st_nt(p, r); }
  __device__ static Vec8 zero() {
    Vec8 v;
    v.r = u32x4{0u, 0u, 0u, 0u};
    return v;
  }
  __device__ bf16x8 to_bf16() const { return __builtin_bit_cast(bf16x8, r); }
  __device__ bf16 get(int i) const { return __builtin_bit_cast(bf16x8, r)[i]; }
  __device__ void set(int i, bf16 x) {
    bf16x8 t = __builtin_bit_cast(bf16x8, r);
    t[i] = x;
    r = __builtin_bit_cast(u32x4, t);
  }
};

template <>
struct Vec8<float> {
  f32x4 a, b;
  __device__ static Vec8 load(const float* p) {
    Vec8 v;
    v.a = *reinterpret_cast<const f32x4*>(p);
    v.b = *reinterpret_cast<const f32x4*>(p + 4);
    return v;
  }
  __device__ void store(float* p) const {
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
  __device__ static Vec8 load_nt(const float* p) {
    Vec8 v;
    v.a = __builtin_bit_cast(f32x4, ld_nt(p));
    v.b = __builtin_bit_cast(f32x4, ld_nt(p + 4));
    return v;
  }
  __device__ void store_nt(float* p) const {
    st_nt(p, __builtin_bit_cast(u32x4, a));
    st_nt(p + 4, __builtin_bit_cast(u32x4, b));
  }
  __device__ static Vec8 zero() {
    Vec8 v;
    v.a = f32x4{0.f, 0.f, 0.f, 0.f};
    v.b = v.a;
    return v;
  }
  // Round-to-nearest-even, the rounding of torch's .to(torch.bfloat16).
  __device__ bf16x8 to_bf16() const {
    bf16x8 o;
    o[0] = (bf16)a[0]; o[1] = (bf16)a[1]; o[2] = (bf16)a[2]; o[3] = (bf16)a[3];
    o[4] = (bf16)b[0]; o[5] = (bf16)b[1]; o[6] = (bf16)b[2]; o[7] = (bf16)b[3];
    return o;
  }
  // Round-to-nearest-even, the rounding of torch's .to(torch.float16).
  __device__ f16x8 to_f16() const {
    f16x8 o;
    o[0] = (f16)a[0]; o[1] = (f16)a[1]; o[2] = (f16)a[2]; o[3] = (f16)a[3];
    o[4] = (f16)b[0]; o[5] = (f16)b[1]; o[6] = (f16)b[2]; o[7] = (f16)b[3];
    return o;
  }
  __device__ float get(int i) const { return i < 4 ? a[i] : b[i - 4]; }
  __device__ void set(int i, float x) {
    if (i < 4) a[i] = x; else b[i - 4] = x;
  }
};

// IEEE binary16 (fp16 attention: f16 pools, queries and outputs)
template <>
struct Vec8<f16> {
  u32x4 r;
  __device__ static Vec8 load(const f16* p) {
    Vec8 v;
    v.r = *reinterpret_cast<const u32x4*>(p);
    return v;
  }
  __device__ void store(f16* p) const { *reinterpret_cast<u32x4*>(p) = r; }
  __device__ static Vec8 zero() {
    Vec8 v;
    v.r = u32x4{0u, 0u, 0u, 0u};
    return v;
  }
  __device__ f16x8 to_f16() const { return __builtin_bit_cast(f16x8, r); }
  __device__ f16 get(int i) const { return __builtin_bit_cast(f16x8, r)[i]; }
  __device__ void set(int i, f16 x) {
    f16x8 t = __builtin_bit_cast(f16x8, r);
    t[i] = x;
    r = __builtin_bit_cast(u32x4, t);
  }
};

// ---- fp8 e4m3fn (OCP) encoding ------------------------------------------------------------
// Software round-to-nearest-even encoder for |x| <= 448 (callers clamp first).  e4m3fn:
// bias 7, max normal 448 (0x7e), min normal 2^-6, subnormal step 2^-9, no infinities.
__device__ inline uint8_t f32_to_e4m3(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  uint32_t sign = (u >> 24) & 0x80u;
  float ax = __builtin_fabsf(x);
  if (!(ax == ax)) return (uint8_t)(sign | 0x7f);  // NaN
  if (ax >= 448.0f) return (uint8_t)(sign | 0x7e);
  uint32_t au = __builtin_bit_cast(uint32_t, ax);
  int exp = (int)(au >> 23) - 127;
  uint32_t code;
  if (exp < -6) {
    // subnormal range: value = m * 2^-9, m in [0, 8]; round ax * 512 to nearest even integer
    float m = ax * 512.0f;                       // exact (power-of-two scaling)
    float r = __builtin_rintf(m);                // RNE under the default rounding mode
    code = (uint32_t)r;                          // r == 8 encodes the min normal 2^-6 (0x08)
  } else {
    uint32_t mant = au & 0x7fffffu;
    uint32_t keep = mant >> 20;                  // top 3 mantissa bits
    uint32_t rest = mant & 0xfffffu;             // 20 dropped bits
    uint32_t half = 0x80000u;
    uint32_t e = (uint32_t)(exp + 7);
    code = (e << 3) | keep;
    if (rest > half || (rest == half && (keep & 1u))) code += 1;  // carry may bump exponent
    if (code > 0x7eu) code = 0x7eu;              // saturate (cannot pass 448 after clamp)
  }
  return (uint8_t)(sign | code);
}

__device__ inline float e4m3_to_f32(uint8_t c) {
  uint32_t sign = (uint32_t)(c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xfu;
  uint32_t m = c & 0x7u;
  float mag;
  if (e == 0) {
    mag = (float)m * (1.0f / 512.0f);
  } else {
    mag = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  }
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, mag) | sign);
}

}  // namespace skv
