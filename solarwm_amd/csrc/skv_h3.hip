// MiniMax-H3's per-segment transforms on gfx950: rotate-half MM-RoPE on head channels [0, 96)
// and the camera PRoPE projection of channels [96, 128), one pass over a token-major bf16
// tensor (skv_h3_rope_prope).  Reference: fused_prope.py:196-255 (rope_prope) and :30-93
// (prope_project), applied around attention by sgf_attention.py:192-203 and :580-659.
#include <stdint.h>

#include "skv_common.h"

namespace skv {

namespace {

struct H3Args {
  const bf16* x;
  bf16* out;
  int64_t x_sb, x_st, x_sh, o_sb, o_st, o_sh;
  const void* cos;
  const void* sin;
  int64_t tab_st;
  const void* m;
  int64_t m_sb, m_st;
  int batch, rows, heads;
};

// A block moves kPairs (row, head) pairs of 256 B, heads fastest, so that a contiguous
// [rows][heads][128] tensor is read and written as one 16 KB run per block; 16 threads per
// pair, kIter pairs per thread with every load issued before the first store.
constexpr int kIter = 4;
constexpr int kPairs = 16 * kIter;

// Every product and sum below is rounded where the reference rounds it: no contraction into
// FMAs (a fused x2 s1 + t would skip the bf16 rounding of the product).
#pragma clang fp contract(off)

__device__ inline float bf16r(float x) { return (float)(bf16)x; }

typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// bf16 rounding of two values with one packed convert (nearest even, as bf16r)
__device__ inline void bf16r2(float& a, float& b) {
  const uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  a = __uint_as_float(r << 16);
  b = __uint_as_float(r & 0xffff0000u);
}

// 8 table / matrix values as floats rounded to bf16 (bf16 inputs are exact already)
template <typename T>
__device__ inline void to_f32r(const Vec8<T>& v, float (&o)[8]) {
  if constexpr (sizeof(T) == 2) {
    const u32x4 r = v.r;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      o[2 * w] = __uint_as_float(r[w] << 16);
      o[2 * w + 1] = __uint_as_float(r[w] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      o[e] = v.get(e);
      o[e + 1] = v.get(e + 1);
      bf16r2(o[e], o[e + 1]);
    }
  }
}

__device__ inline void unpack8(const u32x4& r, float (&o)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    o[2 * w] = __uint_as_float(r[w] << 16);
    o[2 * w + 1] = __uint_as_float(r[w] & 0xffff0000u);
  }
}

__device__ inline u32x4 pack8(const float (&y)[8]) {
  bf16x8 b;
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = (bf16)y[i];
  return __builtin_bit_cast(u32x4, b);
}

// grid ceil(B * rows * H / kPairs), block 256: thread (j, v) owns channels 8v .. 8v+7 of pairs
// blockIdx.x * kPairs + 16 i + j, i < kIter (pair = (b * rows + row) * H + h).  Every load of
// the block (features, the row's cos / sin at the thread's channels, the row's matrix) is
// issued before the barrier and every store follows it, so out may be x.  A rotary vector
// (v < 12) takes its partner half (v +- 6) from the partner lane, which loaded it.
// DENSE: x and out are contiguous [B][rows][heads][128], so pair p starts at element 128 p.
template <typename TT, typename MT, bool ROPE, bool CAM, bool DENSE>
__global__ __launch_bounds__(256) void h3_rope_prope_kernel(H3Args a) {
  const int tid = threadIdx.x, j = tid >> 4, v = tid & 15;
  const int n_pairs = a.batch * a.rows * a.heads;  // < 2^31 (checked on the host)
  int row_of[kIter], b_of[kIter], h_of[kIter], pair_of[kIter];
  u32x4 own[kIter];
  Vec8<TT> tc[kIter], ts[kIter];
  Vec8<MT> m0[kIter], m1[kIter];
#pragma unroll
  for (int i = 0; i < kIter; ++i) {
    const int pair = (int)blockIdx.x * kPairs + 16 * i + j;
    own[i] = u32x4{0u, 0u, 0u, 0u};
    row_of[i] = -1;
    if (pair < n_pairs) {
      const int h = pair % a.heads, br = pair / a.heads;
      const int row = br % a.rows, b = br / a.rows;
      row_of[i] = row;
      pair_of[i] = pair;
      b_of[i] = b;
      h_of[i] = h;
      const int64_t xo = DENSE ? (int64_t)pair * kHeadDim
                               : (int64_t)b * a.x_sb + (int64_t)h * a.x_sh + (int64_t)row * a.x_st;
      own[i] = *reinterpret_cast<const u32x4*>(a.x + xo + 8 * v);
      if (ROPE && v < 12) {
        tc[i] = Vec8<TT>::load(static_cast<const TT*>(a.cos) + (int64_t)row * a.tab_st + 8 * v);
        ts[i] = Vec8<TT>::load(static_cast<const TT*>(a.sin) + (int64_t)row * a.tab_st + 8 * v);
      }
      if (CAM && v >= 12) {
        const MT* mp = static_cast<const MT*>(a.m) + (int64_t)b * a.m_sb + (int64_t)row * a.m_st;
        m0[i] = Vec8<MT>::load(mp);
        m1[i] = Vec8<MT>::load(mp + 8);
      }
    }
  }
  __syncthreads();
  const int partner = (tid & 63 & ~15) | (v < 6 ? v + 6 : v < 12 ? v - 6 : v);
#pragma unroll
  for (int i = 0; i < kIter; ++i) {
    u32x4 part = own[i];
    if constexpr (ROPE) {  // every lane takes part (the shuffle is wave-wide)
#pragma unroll
      for (int w = 0; w < 4; ++w) part[w] = (uint32_t)__shfl((int)own[i][w], partner, 64);
    }
    if (row_of[i] < 0) continue;
    const int row = row_of[i], b = b_of[i], h = h_of[i];
    u32x4 res = own[i];
    if (ROPE && v < 12) {
      // y1 = x1 c1 + (-x2) s1 (v < 6: x1 own, x2 partner); y2 = x2 c2 + x1 s2 (x2 own, x1
      // partner); negating the bf16 partner is exact
      float xo[8], xp[8], c[8], sn[8], p[8], q[8], y[8];
      unpack8(own[i], xo);
      unpack8(part ^ (v < 6 ? u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u}
                            : u32x4{0u, 0u, 0u, 0u}), xp);
      to_f32r(tc[i], c);
      to_f32r(ts[i], sn);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = xo[e] * c[e];
        q[e] = xp[e] * sn[e];
      }
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        bf16r2(p[e], p[e + 1]);
        bf16r2(q[e], q[e + 1]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = p[e] + q[e];
      res = pack8(y);
    }
    if (CAM && v >= 12) {
      float m[16], xo[8], y[8];
      {
        float ma[8], mb[8];
        to_f32r(m0[i], ma);
        to_f32r(m1[i], mb);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          m[e] = ma[e];
          m[8 + e] = mb[e];
        }
      }
      unpack8(own[i], xo);
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* mi = m + 4 * r;
          const float* xv = xo + 4 * g;
          // bf16 x bf16 products are exact in fp32: the sum order alone fixes the result
          y[4 * g + r] = ((mi[0] * xv[0] + mi[1] * xv[1]) + mi[2] * xv[2]) + mi[3] * xv[3];
        }
      res = pack8(y);
    }
    const int64_t oo = DENSE ? (int64_t)pair_of[i] * kHeadDim
                             : (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)row * a.o_st;
    *reinterpret_cast<u32x4*>(a.out + oo + 8 * v) = res;
  }
}

template <typename TT, typename MT, bool DENSE>
void launch_h3(const H3Args& a, bool rope, bool cam, dim3 grid, hipStream_t s) {
  if (rope && cam)
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, true, true, DENSE>), grid, dim3(256), 0, s, a);
  else if (rope)
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, true, false, DENSE>), grid, dim3(256), 0, s, a);
  else if (cam)
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, false, true, DENSE>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, false, false, DENSE>), grid, dim3(256), 0, s, a);
}

template <typename TT, typename MT>
void launch_h3(const H3Args& a, bool rope, bool cam, bool dense, dim3 grid, hipStream_t s) {
  if (dense)
    launch_h3<TT, MT, true>(a, rope, cam, grid, s);
  else
    launch_h3<TT, MT, false>(a, rope, cam, grid, s);
}

// byte extent [lo, hi) of a [batch][rows][heads][128] view of 2-byte elements
void extent(const void* p, int64_t sb, int64_t st, int64_t sh, int batch, int rows, int heads,
            uintptr_t& lo, uintptr_t& hi) {
  lo = reinterpret_cast<uintptr_t>(p);
  hi = lo + 2 * ((batch - 1) * sb + (rows - 1) * st + (heads - 1) * sh + kHeadDim);
}

}  // namespace

}  // namespace skv

using namespace skv;

extern "C" int skv_h3_rope_prope(const skv_h3_xform_desc* d, skv_stream_t stream) {
  clear_error();
  if (!d || !d->x || !d->out) {
    set_error("skv_h3_rope_prope: null descriptor, x or out");
    return SKV_E_ARG;
  }
  if (d->head_dim != kHeadDim) {
    set_error("skv_h3_rope_prope: head_dim=%d unsupported (built for %d)", d->head_dim, kHeadDim);
    return SKV_E_UNSUPPORTED;
  }
  if (d->batch <= 0 || d->rows < 0 || d->heads <= 0 ||
      (int64_t)d->batch * d->rows * d->heads + kPairs >= ((int64_t)1 << 31)) {
    set_error("skv_h3_rope_prope: bad sizes (batch=%d rows=%d heads=%d)", d->batch, d->rows,
              d->heads);
    return SKV_E_ARG;
  }
  if ((d->cos == nullptr) != (d->sin == nullptr)) {
    set_error("skv_h3_rope_prope: give both cos and sin, or neither");
    return SKV_E_ARG;
  }
  const bool rope = d->cos != nullptr, cam = d->matrix != nullptr;
  if ((rope && d->table_dtype != SKV_BF16 && d->table_dtype != SKV_F32) ||
      (cam && d->matrix_dtype != SKV_BF16 && d->matrix_dtype != SKV_F32)) {
    set_error("skv_h3_rope_prope: tables and matrices must be bf16 or f32");
    return SKV_E_UNSUPPORTED;
  }
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (d->x_sb % 8 || d->x_st % 8 || d->x_sh % 8 || d->out_sb % 8 || d->out_st % 8 ||
      d->out_sh % 8 || !a16(d->x) || !a16(d->out) || d->x_sb < 0 || d->x_st < 0 ||
      d->x_sh < 0 || d->out_sb < 0 || d->out_st < 0 || d->out_sh < 0) {
    set_error("skv_h3_rope_prope: x / out strides must be non-negative multiples of 8 elements "
              "and the pointers 16-byte aligned");
    return SKV_E_ARG;
  }
  if (rope) {
    const int esz = d->table_dtype == SKV_F32 ? 4 : 2;
    if (d->table_stride < 96 || d->table_stride % 8 ||
        reinterpret_cast<uintptr_t>(d->cos) % (8 * esz) ||
        reinterpret_cast<uintptr_t>(d->sin) % (8 * esz)) {
      set_error("skv_h3_rope_prope: cos / sin rows need >= 96 elements, a stride that is a "
                "multiple of 8 and 8-element aligned pointers");
      return SKV_E_ARG;
    }
  }
  if (cam) {
    const int esz = d->matrix_dtype == SKV_F32 ? 4 : 2;
    if (d->matrix_st < 16 || d->matrix_st % 8 || d->matrix_sb < 0 || d->matrix_sb % 8 ||
        reinterpret_cast<uintptr_t>(d->matrix) % (8 * esz)) {
      set_error("skv_h3_rope_prope: matrix rows need 16 elements, strides that are multiples "
                "of 8 and an 8-element aligned pointer");
      return SKV_E_ARG;
    }
  }
  if (d->rows == 0) return SKV_OK;
  const bool same = d->x == d->out && d->x_sb == d->out_sb && d->x_st == d->out_st &&
                    d->x_sh == d->out_sh;
  if (!same) {
    uintptr_t xl, xh, ol, oh;
    extent(d->x, d->x_sb, d->x_st, d->x_sh, d->batch, d->rows, d->heads, xl, xh);
    extent(d->out, d->out_sb, d->out_st, d->out_sh, d->batch, d->rows, d->heads, ol, oh);
    if (xl < oh && ol < xh) {
      set_error("skv_h3_rope_prope: out overlaps x without being x itself");
      return SKV_E_ARG;
    }
  }
  H3Args a{static_cast<const bf16*>(d->x), static_cast<bf16*>(d->out), d->x_sb, d->x_st,
           d->x_sh, d->out_sb, d->out_st, d->out_sh, d->cos, d->sin, d->table_stride,
           d->matrix, d->matrix_sb, d->matrix_st, d->batch, d->rows, d->heads};
  const int64_t n_pairs = (int64_t)d->batch * d->rows * d->heads;
  const dim3 grid((unsigned)((n_pairs + kPairs - 1) / kPairs));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool tf = rope && d->table_dtype == SKV_F32, mf = cam && d->matrix_dtype == SKV_F32;
  const int64_t st = (int64_t)d->heads * kHeadDim, sb = st * d->rows;
  const bool dense = d->x_sh == kHeadDim && d->x_st == st && (d->batch == 1 || d->x_sb == sb) &&
                     d->out_sh == kHeadDim && d->out_st == st && (d->batch == 1 || d->out_sb == sb);
  if (tf) {
    if (mf) launch_h3<float, float>(a, rope, cam, dense, grid, s);
    else launch_h3<float, bf16>(a, rope, cam, dense, grid, s);
  } else {
    if (mf) launch_h3<bf16, float>(a, rope, cam, dense, grid, s);
    else launch_h3<bf16, bf16>(a, rope, cam, dense, grid, s);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("skv_h3_rope_prope: launch failed: %s", hipGetErrorString(e));
    return SKV_E_LAUNCH;
  }
  return SKV_OK;
}
