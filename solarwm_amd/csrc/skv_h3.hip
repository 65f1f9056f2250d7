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
  int rows, heads;
};

constexpr int kRowsPerBlock = 16;  // 16 rows x 16 vectors of 8 channels = 256 threads

__device__ inline float bf16r(float x) { return (float)(bf16)x; }

// 8 consecutive table values as floats rounded to bf16 (the reference rounds f32 tables)
template <typename TT>
__device__ inline void load8r(const TT* p, float (&o)[8]) {
  const Vec8<TT> v = Vec8<TT>::load(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = bf16r((float)v.get(i));
}

__device__ inline void unpack8(const u32x4& r, float (&o)[8]) {
  const bf16x8 b = __builtin_bit_cast(bf16x8, r);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (float)b[i];
}

__device__ inline u32x4 pack8(const float (&y)[8]) {
  bf16x8 b;
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = (bf16)y[i];
  return __builtin_bit_cast(u32x4, b);
}

// grid (ceil(rows / 16), heads, batch), block 256: thread (r, v) owns channels 8v .. 8v+7 of
// row blockIdx.x * 16 + r.  Rotary vectors (v < 12) also read their partner half (v +- 6) and
// the row's cos / sin at their own channels; camera vectors (v >= 12) read the row's matrix.
// Every load of the block precedes the barrier and every store follows it, so out may be x.
template <typename TT, typename MT, bool ROPE, bool CAM>
__global__ __launch_bounds__(256) void h3_rope_prope_kernel(H3Args a) {
  const int tid = threadIdx.x, r = tid >> 4, v = tid & 15;
  const int row = blockIdx.x * kRowsPerBlock + r, h = blockIdx.y, b = blockIdx.z;
  const bool live = row < a.rows;
  const bf16* xr = a.x + (int64_t)b * a.x_sb + (int64_t)h * a.x_sh + (int64_t)row * a.x_st;
  u32x4 own = u32x4{0u, 0u, 0u, 0u}, part = own;
  float c[8], s[8], m[16];
  if (live) {
    own = *reinterpret_cast<const u32x4*>(xr + 8 * v);
    if constexpr (ROPE) {
      if (v < 12) {
        const int p = v < 6 ? v + 6 : v - 6;
        part = *reinterpret_cast<const u32x4*>(xr + 8 * p);
        load8r(static_cast<const TT*>(a.cos) + (int64_t)row * a.tab_st + 8 * v, c);
        load8r(static_cast<const TT*>(a.sin) + (int64_t)row * a.tab_st + 8 * v, s);
      }
    }
    if constexpr (CAM) {
      if (v >= 12) {
        const MT* mp = static_cast<const MT*>(a.m) + (int64_t)b * a.m_sb + (int64_t)row * a.m_st;
        float m0[8], m1[8];
        load8r(mp, m0);
        load8r(mp + 8, m1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          m[i] = m0[i];
          m[8 + i] = m1[i];
        }
      }
    }
  }
  __syncthreads();
  if (!live) return;
  u32x4 res = own;
  if (ROPE && v < 12) {
    float xo[8], xp[8], y[8];
    unpack8(own, xo);
    unpack8(part, xp);
    if (v < 6) {  // y1 = x1 c1 - x2 s1 (x1 own, x2 partner)
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = bf16r(bf16r(xo[i] * c[i]) + bf16r(-xp[i] * s[i]));
    } else {      // y2 = x2 c2 + x1 s2 (x2 own, x1 partner)
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = bf16r(bf16r(xo[i] * c[i]) + bf16r(xp[i] * s[i]));
    }
    res = pack8(y);
  }
  if (CAM && v >= 12) {
    float xo[8], y[8];
    unpack8(own, xo);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float* mi = m + 4 * i;
        const float* xv = xo + 4 * g;
        // bf16 x bf16 products are exact in fp32: the sum order alone fixes the result
        y[4 * g + i] = ((mi[0] * xv[0] + mi[1] * xv[1]) + mi[2] * xv[2]) + mi[3] * xv[3];
      }
    res = pack8(y);
  }
  bf16* orow = a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)row * a.o_st;
  *reinterpret_cast<u32x4*>(orow + 8 * v) = res;
}

template <typename TT, typename MT>
void launch_h3(const H3Args& a, bool rope, bool cam, dim3 grid, hipStream_t s) {
  if (rope && cam)
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, true, true>), grid, dim3(256), 0, s, a);
  else if (rope)
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, true, false>), grid, dim3(256), 0, s, a);
  else if (cam)
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, false, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((h3_rope_prope_kernel<TT, MT, false, false>), grid, dim3(256), 0, s, a);
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
  if (d->batch <= 0 || d->rows < 0 || d->heads <= 0 || d->batch > 65535 || d->heads > 65535) {
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
           d->matrix, d->matrix_sb, d->matrix_st, d->rows, d->heads};
  const dim3 grid((unsigned)((d->rows + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)d->heads,
                  (unsigned)d->batch);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool tf = rope && d->table_dtype == SKV_F32, mf = cam && d->matrix_dtype == SKV_F32;
  if (tf) {
    if (mf) launch_h3<float, float>(a, rope, cam, grid, s);
    else launch_h3<float, bf16>(a, rope, cam, grid, s);
  } else {
    if (mf) launch_h3<bf16, float>(a, rope, cam, grid, s);
    else launch_h3<bf16, bf16>(a, rope, cam, grid, s);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("skv_h3_rope_prope: launch failed: %s", hipGetErrorString(e));
    return SKV_E_LAUNCH;
  }
  return SKV_OK;
}
