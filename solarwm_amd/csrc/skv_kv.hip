// Frame-slot K/V movement kernels for gfx950: append (token-major chunk -> pool slots, with
// optional fp8 e4m3fn quantisation) and gather (pool slots -> token-major frames).
//
// The reference moves whole K/V windows on every forward (clone + memmove + slice-assign,
// solar/backends/wan22/runtime/modeling/causal_model.py:1054-1080, :2881-2898).  Here a frame
// is written once into a slot and never moved again; eviction is a slot-table update on the
// host.  Both kernels are HBM-bound byte movers: one workgroup moves one 64-token tile of one
// (frame, batch, head); K rows move as 16 B vectors, V is transposed in registers, 8 tokens x 8
// channels per thread, so the pool keeps V channel-major (tokens contiguous), which is what the
// attention kernel's PV product reads.
#include <cstdlib>

#include "skv_common.h"

namespace skv {

struct AppendArgs {
  const void* ksrc;
  const void* vsrc;
  int64_t s_sb, s_st, s_sh;  // element strides of the token-major source
  void* kpool;
  void* vpool;
  float* kscale;
  float* vscale;
  int64_t slot_stride;  // elements per slot in each pool (B*H*Tp*D)
  int B, H, T, Tp, n_frames, src_frame0, ntiles;
  // RoPE copy (bf16/fp32 pools): krpool receives K with the height/width pairs of Wan's RoPE
  // applied (rope_hw: cos, sin per (h, pair) then per (w, pair)); nullptr = no copy
  void* krpool;
  const float* rope_hw;
  int gh, gw;
  // PRoPE (needs krpool): kv_xf [n_frames][B][16] = P^-1 (row-major 4x4) of each written frame's
  // camera; krpool's spatial channel groups (44..127, after their RoPE) and every group of
  // vrpool (V, laid out as vpool) receive P^-1 x per group of 4 channels
  void* vrpool;
  const float* kv_xf;
  // RMSNorm of K (the reference's norm_k before the cache write): source token t of stream b
  // is scaled by krms[b * krms_sb + t] (1 / RMS over the token's H x D row) and channel
  // h*D + c by kw[h*D + c], in fp32, then rounded once to the source dtype; nullptr = raw K
  const float* krms;
  int64_t krms_sb;
  const float* kw;
  // fp8 pools: the copies' scales ([n_slots][B][H], absmax / 448 of each written copy)
  float* krscale;
  float* vrscale;
  int32_t slots[SKV_MAX_APPEND_FRAMES];
};

// K row [col, col+8) of source token `tok` (stream b, head h) through RMSNorm: x * rms * w,
// fp32 products, one rounding to E (the value the raw pool stores and everything derives from)
template <typename E>
__device__ inline void norm8(Vec8<E>& v, const AppendArgs& a, int b, int h, int64_t tok, int col) {
  const float r = a.krms[(int64_t)b * a.krms_sb + tok];
  const float* w = a.kw + h * kHeadDim + col;
#pragma unroll
  for (int e = 0; e < 8; ++e) v.set(e, (E)((float)v.get(e) * r * w[e]));
}

// Wan splits a head's 64 complex channel pairs (2i, 2i+1) into 22 temporal, 21 height and 21
// width pairs (causal_model.py:1855-1866).
constexpr int kRopeT = 22, kRopeHW = 21;

// Rotate the spatial pairs among channels [col, col+8) of token t (grid width gw): pair p in
// [22, 43) turns by the angle of row h = t / gw, p in [43, 64) by that of column w = t % gw.
__device__ inline void rope_spatial8(Vec8<float>& v, int col, int t, int gh, int gw, const float* tab) {
  if (col + 8 <= 2 * kRopeT) return;
  const int hq = t / gw, wq = t - hq * gw;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int p = col / 2 + m;
    if (p < kRopeT) continue;
    const int idx = p < kRopeT + kRopeHW ? hq * kRopeHW + (p - kRopeT) : (gh + wq) * kRopeHW + (p - kRopeT - kRopeHW);
    const float c = tab[2 * idx], sn = tab[2 * idx + 1];
    const float x = v.get(2 * m), y = v.get(2 * m + 1);
    v.set(2 * m, x * c - y * sn);
    v.set(2 * m + 1, x * sn + y * c);
  }
}

// y[4g .. 4g+4) <- m (row-major 4x4) x y[4g .. 4g+4)
__device__ inline void xform4(Vec8<float>& y, int g, const float* m) {
  const float x0 = y.get(4 * g), x1 = y.get(4 * g + 1), x2 = y.get(4 * g + 2), x3 = y.get(4 * g + 3);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    y.set(4 * g + i, fmaf(m[4 * i], x0, fmaf(m[4 * i + 1], x1, fmaf(m[4 * i + 2], x2, m[4 * i + 3] * x3))));
}

template <typename E>
__device__ inline Vec8<float> to_f32(const Vec8<E>& v) {
  Vec8<float> y;
#pragma unroll
  for (int e = 0; e < 8; ++e) y.set(e, (float)v.get(e));
  return y;
}

template <typename E>
__device__ inline Vec8<E> from_f32(const Vec8<float>& y) {
  Vec8<E> v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v.set(e, (E)y.get(e));
  return v;
}

// 8x8 transpose of 16-bit elements held as 8 rows of 4 x u32 (row r = token, word c/2 half c%2
// = channel c): out[c].word[w] = (in[2w] half c, in[2w+1] half c).
__device__ inline void transpose8x8_b16(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a = in[2 * w][c >> 1], b = in[2 * w + 1][c >> 1];
      // v_perm_b32 selector: bytes 0-3 come from the second operand, 4-7 from the first
      out[c][w] = (c & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u)   // hi halves
                          : __builtin_amdgcn_perm(b, a, 0x05040100u);  // lo halves
    }
}

// grid.x = n_frames * B * H * ntiles (ntiles = Tp / 64), block = 256.  Threads 0-127 copy the
// 64 K rows (16 B vectors); threads 128-255 each move one 8-token x 8-channel block of V,
// transposed in registers, so V^T rows are written as 16 B vectors without an LDS stage.
// Rows past T are written as zeros.
// XM: 0 = pools only, 1 = + RoPE copy of K (krpool), 2 = + PRoPE copies of K and V
template <typename E, int XM>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
  int wg = blockIdx.x;
  const int t = wg % a.ntiles;
  wg /= a.ntiles;
  const int h = wg % a.H;
  wg /= a.H;
  const int b = wg % a.B;
  const int f = wg / a.B;
  const int64_t slot = a.slots[f];
  const int tid = threadIdx.x;
  const int tok0 = t * kTile;
  const int64_t src_base = (int64_t)b * a.s_sb + (int64_t)h * a.s_sh +
                           (int64_t)(a.src_frame0 + f) * a.T * a.s_st;
  if (tid < 128) {
    const E* __restrict__ ks = static_cast<const E*>(a.ksrc);
    E* __restrict__ kp = static_cast<E*>(a.kpool) + slot * a.slot_stride +
                         ((int64_t)(b * a.H + h) * a.Tp + tok0) * kHeadDim;
    // 64 rows x 16 vec8 = 1024 vec8, 8 per thread.  All eight loads are issued before any store
    // (rows past T read the frame's last row and are then zeroed, so no load sits behind a
    // branch): the source is usually cold in HBM, and loads interleaved with stores would wait
    // for each other's round trips.
    const int col = (tid & 15) * 8;
    Vec8<E> kv[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int row = (tid >> 4) + 8 * r;
      const int srow = min(tok0 + row, a.T - 1);
      kv[r] = Vec8<E>::load_nt(ks + src_base + (int64_t)srow * a.s_st + col);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int row = (tid >> 4) + 8 * r;
      const bool live = tok0 + row < a.T;
      if (!live) kv[r] = Vec8<E>::zero();
      if (a.krms && live) norm8(kv[r], a, b, h, (int64_t)(a.src_frame0 + f) * a.T + tok0 + row, col);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int row = (tid >> 4) + 8 * r;
      const bool live = tok0 + row < a.T;
      Vec8<E> kv_r = kv[r];
      kv_r.store_nt(kp + row * kHeadDim + col);
      if constexpr (XM > 0) {
        if (live && col + 8 > 2 * kRopeT) {
          Vec8<float> y = to_f32(kv_r);
          rope_spatial8(y, col, tok0 + row, a.gh, a.gw, a.rope_hw);
          if constexpr (XM == 2) {
            const float* m = a.kv_xf + ((int64_t)f * a.B + b) * 16;
#pragma unroll
            for (int gg = 0; gg < 2; ++gg)
              if (col + 4 * gg >= 2 * kRopeT) xform4(y, gg, m);
          }
          kv_r = from_f32<E>(y);
        }
        kv_r.store_nt(static_cast<E*>(a.krpool) + (kp - static_cast<E*>(a.kpool)) + row * kHeadDim + col);
      }
    }
    return;
  }
  const E* __restrict__ vs = static_cast<const E*>(a.vsrc);
  E* __restrict__ vp = static_cast<E*>(a.vpool) + slot * a.slot_stride +
                       (int64_t)(b * a.H + h) * kHeadDim * a.Tp + tok0;
  const int i = tid - 128;
  // tokens tb*8.., channels db*8..: each wave instruction covers 128 B of 8 token rows on the
  // read side and 128 B of 8 V^T rows on the write side
  const int tb = i & 7, db = i >> 3;
  if constexpr (sizeof(E) == 2) {
    u32x4 in[8], out[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {  // unconditional loads (clamped row), zeroed past T
      const int tok = min(tok0 + tb * 8 + r, a.T - 1);
      in[r] = ld_nt(vs + src_base + (int64_t)tok * a.s_st + db * 8);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r)
      if (tok0 + tb * 8 + r >= a.T) in[r] = u32x4{0u, 0u, 0u, 0u};
    transpose8x8_b16(in, out);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      st_nt(vp + (int64_t)(db * 8 + c) * a.Tp + tb * 8, out[c]);
    if constexpr (XM == 2) {
      // P^-1 per token on both channel groups, then the same transpose into vrpool (rows past
      // T stay zero)
      const float* m = a.kv_xf + ((int64_t)f * a.B + b) * 16;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        Vec8<bf16> x;
        x.r = in[r];
        Vec8<float> y = to_f32(x);
        xform4(y, 0, m);
        xform4(y, 1, m);
        in[r] = from_f32<bf16>(y).r;
      }
      transpose8x8_b16(in, out);
      E* vx = static_cast<E*>(a.vrpool) + (vp - static_cast<E*>(a.vpool));
#pragma unroll
      for (int c = 0; c < 8; ++c)
        st_nt(vx + (int64_t)(db * 8 + c) * a.Tp + tb * 8, out[c]);
    }
  } else {
    Vec8<E> in[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int tok = min(tok0 + tb * 8 + r, a.T - 1);
      in[r] = Vec8<E>::load_nt(vs + src_base + (int64_t)tok * a.s_st + db * 8);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r)
      if (tok0 + tb * 8 + r >= a.T) in[r] = Vec8<E>::zero();
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      Vec8<E> o;
#pragma unroll
      for (int r = 0; r < 8; ++r) o.set(r, in[r].get(c));
      o.store_nt(vp + (int64_t)(db * 8 + c) * a.Tp + tb * 8);
    }
  }
}

// fp8 append with the frame held on chip (bf16 sources, Tp <= 64 * kFp8OnChip): one
// 1024-thread workgroup per (frame, batch, head, K|V); thread t owns chunk j = 16 B of row
// 64 j + t / 16, channels (t % 16) * 8 .. +8.  Every chunk of the frame is loaded at once (one
// HBM read, all loads in flight): the first kFp8RegChunks into registers, the rest straight into
// LDS (buffer_load ... lds, 16 KB per chunk).  The workgroup reduces the absmax and the codes
// come from the hardware e4m3 convert, which on clamped inputs gives exactly the
// round-to-nearest-even codes of f32_to_e4m3.  V^T tiles go through a double-buffered LDS tile
// (one barrier per tile).
constexpr int kFp8RegChunks = 18;
constexpr int kFp8LdsChunks = 7;
constexpr int kFp8OnChip = kFp8RegChunks + kFp8LdsChunks;
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ inline uint32_t e4m3x4(float a, float b, float c, float d) {
  int v = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  v = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, v, true);
  return (uint32_t)v;
}

__device__ inline u32x2 quant8(const u32x4& r, float inv) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(r[i] << 16);
    f[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = fminf(fmaxf(f[i] * inv, -448.0f), 448.0f);
  return u32x2{e4m3x4(f[0], f[1], f[2], f[3]), e4m3x4(f[4], f[5], f[6], f[7])};
}

// |x| of a bf16 is its bits & 0x7fff, and non-negative bf16 order as integers: the absmax runs
// on packed 16-bit integer maxima (no unpacking to fp32, which would double the live state)
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ inline u16x2 absmax8(const u32x4& r, u16x2 m) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, r[i] & 0x7fff7fffu));
  return m;
}

__global__ __launch_bounds__(1024) void append_fp8_reg_kernel(AppendArgs a) {
  constexpr int kRowT = kTile + 4;  // V^T tile row: 64 tokens + 4 bytes of skew
  constexpr int kChunkBytes = 1024 * 16;
  __shared__ float red[32];
  __shared__ __attribute__((aligned(16))) uint8_t stage[kFp8LdsChunks * kChunkBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vt8[2][kHeadDim * kRowT];
  int wg = blockIdx.x;
  const int is_v = wg & 1;
  wg >>= 1;
  const int h = wg % a.H;
  wg /= a.H;
  const int b = wg % a.B;
  const int f = wg / a.B;
  const int64_t slot = a.slots[f];
  const int tid = threadIdx.x;
  const int rr = tid >> 4, col = (tid & 15) * 8;
  const bf16* src = static_cast<const bf16*>(is_v ? a.vsrc : a.ksrc) + (int64_t)b * a.s_sb +
                    (int64_t)h * a.s_sh + (int64_t)(a.src_frame0 + f) * a.T * a.s_st;
  // one buffer descriptor per frame: the lane's byte offset is a single VGPR (no 64-bit
  // address per load); the host guarantees the frame spans < 2^31 bytes.  Rows >= T are never
  // loaded (their register chunks are zero, their LDS chunks are masked on read).
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, 0x7fffffff, 0x00020000);
  const uint32_t lane_off = (uint32_t)(rr * a.s_st + col) * 2u;
  const uint32_t row_step = (uint32_t)(kTile * a.s_st) * 2u;
  const int nt = a.ntiles;
  uint8_t* my_stage = stage + tid * 16;
#pragma unroll
  for (int c = 0; c < kFp8LdsChunks; ++c) {
    const int j = kFp8RegChunks + c;
    if (j < nt && kTile * j + rr < a.T)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_void_t*)(stage + c * kChunkBytes + (tid >> 6) * 1024), 16,
          lane_off + j * row_step, 0, 0, 0);
  }
  u32x4 r[kFp8RegChunks];
#pragma unroll
  for (int j = 0; j < kFp8RegChunks; ++j) {
    r[j] = u32x4{0u, 0u, 0u, 0u};
    if (j < nt && kTile * j + rr < a.T)
      r[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off + j * row_step, 0, 0));
  }
  const bool knorm = !is_v && a.krms;
  const int64_t tok_base = (int64_t)(a.src_frame0 + f) * a.T;
  auto normed = [&](u32x4 x, int row) -> u32x4 {
    Vec8<bf16> v;
    v.r = x;
    norm8(v, a, b, h, tok_base + row, col);
    return v.r;
  };
  if (knorm) {
#pragma unroll
    for (int j = 0; j < kFp8RegChunks; ++j)
      if (j < nt && kTile * j + rr < a.T) r[j] = normed(r[j], kTile * j + rr);
  }
  // chunk j of this thread wherever it lives (normalised K), zero for rows >= T
  auto chunk = [&](int j) -> u32x4 {
    if (j < kFp8RegChunks) return r[j];
    const int row = kTile * j + rr;
    if (row >= a.T) return u32x4{0u, 0u, 0u, 0u};
    const u32x4 x = *reinterpret_cast<const u32x4*>(my_stage + (j - kFp8RegChunks) * kChunkBytes);
    return knorm ? normed(x, row) : x;
  };
  u16x2 mm = {0, 0};
#pragma unroll
  for (int j = 0; j < kFp8RegChunks; ++j) mm = absmax8(r[j], mm);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS chunks have landed
#pragma unroll
  for (int j = kFp8RegChunks; j < kFp8OnChip; ++j)
    if (j < nt) mm = absmax8(chunk(j), mm);
  float m = __uint_as_float((uint32_t)(mm[0] > mm[1] ? mm[0] : mm[1]) << 16);
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid < 64) {
    float x = tid < 16 ? red[tid] : 0.f;
    for (int off = 8; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    if (tid == 0) red[16] = x;
  }
  __syncthreads();
  const float amax = red[16];
  const float inv = amax > 0.f ? 448.0f / amax : 0.f;
  if (tid == 0) {
    float* sc = is_v ? a.vscale : a.kscale;
    sc[(slot * a.B + b) * a.H + h] = amax / 448.0f;
  }
  uint8_t* pool = static_cast<uint8_t*>(is_v ? a.vpool : a.kpool) + slot * a.slot_stride +
                  (int64_t)(b * a.H + h) * a.Tp * kHeadDim;
  if (!is_v) {
#pragma unroll
    for (int j = 0; j < kFp8OnChip; ++j)
      if (j < nt)  // rows T..Tp-1 hold zeros -> code 0
        *reinterpret_cast<u32x2*>(pool + (int64_t)(kTile * j + rr) * kHeadDim + col) = quant8(chunk(j), inv);
    return;
  }
  const int d = tid >> 3, tc = (tid & 7) * 8;
#pragma unroll
  for (int j = 0; j < kFp8OnChip; ++j) {
    // `continue`, not `break`: a break keeps the loop from unrolling fully, and r[] then lives
    // in scratch memory (304 bytes per lane) instead of registers
    if (j >= nt) continue;
    uint8_t* buf = vt8[j & 1];
    const u32x2 q = quant8(chunk(j), inv);
#pragma unroll
    for (int i = 0; i < 8; ++i) buf[(col + i) * kRowT + rr] = (uint8_t)(q[i >> 2] >> (8 * (i & 3)));
    __syncthreads();  // buf[j & 1] complete; every read of it two tiles ago is done
    const uint32_t* rd = reinterpret_cast<const uint32_t*>(buf + d * kRowT + tc);
    *reinterpret_cast<u32x2*>(pool + (int64_t)d * a.Tp + kTile * j + tc) = u32x2{rd[0], rd[1]};
  }
}

// fp8 append: one workgroup per (frame, batch, head, K|V).  Pass 1 reduces absmax over the
// frame's T x 128 values; pass 2 re-reads them (L2/MALL resident), quantises with
// inv = 448 / absmax and stores e4m3fn codes (V transposed through LDS).
template <typename E>
__device__ inline float absval8(const Vec8<E>& v, float m) {
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, __builtin_fabsf((float)v.get(i)));
  return m;
}

template <typename E>
__global__ __launch_bounds__(1024) void append_fp8_kernel(AppendArgs a) {
  __shared__ float red[32];
  __shared__ uint8_t vt8[kTile * (kHeadDim + 16)];
  int wg = blockIdx.x;
  const int is_v = wg & 1;
  wg >>= 1;
  const int h = wg % a.H;
  wg /= a.H;
  const int b = wg % a.B;
  const int f = wg / a.B;
  const int64_t slot = a.slots[f];
  const int tid = threadIdx.x;

  const E* src = static_cast<const E*>(is_v ? a.vsrc : a.ksrc);
  src += (int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)(a.src_frame0 + f) * a.T * a.s_st;

  const bool knorm = !is_v && a.krms;
  const int64_t tok_base = (int64_t)(a.src_frame0 + f) * a.T;
  // Pass 1: absmax over T rows x 16 vec8.
  float m = 0.f;
  const int nvec = a.T * 16;
  for (int c = tid; c < nvec; c += 1024) {
    const int row = c >> 4, col = (c & 15) * 8;
    Vec8<E> x = Vec8<E>::load(src + (int64_t)row * a.s_st + col);
    if (knorm) norm8(x, a, b, h, tok_base + row, col);
    m = absval8(x, m);
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid < 64) {
    float x = tid < 16 ? red[tid] : 0.f;
    for (int off = 8; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    if (tid == 0) red[16] = x;
  }
  __syncthreads();
  const float amax = red[16];
  const float inv = amax > 0.f ? 448.0f / amax : 0.f;
  if (tid == 0) {
    float* sc = is_v ? a.vscale : a.kscale;
    sc[(slot * a.B + b) * a.H + h] = amax / 448.0f;
  }

  uint8_t* pool = static_cast<uint8_t*>(is_v ? a.vpool : a.kpool) + slot * a.slot_stride +
                  (int64_t)(b * a.H + h) * a.Tp * kHeadDim;
  // Pass 2: quantise tile by tile (64 tokens), padding rows encode 0.
  for (int t0 = 0; t0 < a.Tp; t0 += kTile) {
    const int c = tid;  // 64 rows x 16 vec8 = 1024 = one vec8 per thread
    const int row = c >> 4, col = (c & 15) * 8;
    const bool live = t0 + row < a.T;
    Vec8<E> v = live ? Vec8<E>::load(src + (int64_t)(t0 + row) * a.s_st + col) : Vec8<E>::zero();
    if (knorm && live) norm8(v, a, b, h, tok_base + t0 + row, col);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float y = fminf(fmaxf((float)v.get(i) * inv, -448.0f), 448.0f);
      uint32_t code = f32_to_e4m3(y);
      if (i < 4) lo |= code << (8 * i); else hi |= code << (8 * (i - 4));
    }
    if (!is_v) {
      *reinterpret_cast<u32x2*>(pool + (int64_t)(t0 + row) * kHeadDim + col) = u32x2{lo, hi};
    } else {
      *reinterpret_cast<u32x2*>(vt8 + row * (kHeadDim + 16) + col) = u32x2{lo, hi};
      __syncthreads();
      // channel d, tokens tc..tc+7 (8 B of codes)
      const int d = c >> 3, tc = (c & 7) * 8;
      uint32_t o0 = 0, o1 = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t code = vt8[(tc + i) * (kHeadDim + 16) + d];
        if (i < 4) o0 |= code << (8 * i); else o1 |= code << (8 * (i - 4));
      }
      *reinterpret_cast<u32x2*>(pool + (int64_t)d * a.Tp + t0 + tc) = u32x2{o0, o1};
      __syncthreads();
    }
  }
}

// fp8 append split over 64-token tiles, for chunks with fewer (frame, batch, head, K|V) units
// than the chip has CUs several times over (C5: 288 units of 25 tiles on 256 CUs, where one
// workgroup per unit runs two rounds of long serial streams).  grid.x = units * ntiles, tile
// fastest, unit u = ((f * B + b) * H + h) * 2 + is_v as in the per-unit kernels.
//  pass 1 (fp8_tile_absmax_kernel): part[blockIdx.x] = absmax of the tile's values (K after its
//          RMSNorm); rows >= T are not read.
//  pass 2 (append_fp8_tile_kernel): amax = max of the unit's tile maxima (the frame's absmax,
//          as the per-unit kernels reduce it), tile 0 stores the scale amax / 448, every tile
//          re-reads its rows (L2/MALL resident after pass 1) and stores their codes; rows T..Tp-1
//          get code 0.  V^T goes through an LDS tile.
// k_only: the grid holds K units only (u = (f * B + b) * H + h), for the RoPE copy of K.
struct TileUnit {
  int t, is_v, h, b, f;
  __device__ TileUnit(const AppendArgs& a, bool k_only) {
    int wg = blockIdx.x;
    t = wg % a.ntiles;
    wg /= a.ntiles;
    is_v = k_only ? 0 : wg & 1;
    if (!k_only) wg >>= 1;
    h = wg % a.H;
    wg /= a.H;
    b = wg % a.B;
    f = wg / a.B;
  }
};

// XM = 0: the raw frames (kpool / vpool).  XM = 1: the RoPE copy of K (krpool), K units only.
// XM = 2: the PRoPE copies, K (krpool: RoPE, then P^-1 on the spatial groups) and V (vrpool:
// P^-1 on every group).  A copy's value is what append_kernel writes into a bf16 / f32 copy
// pool (fp32 arithmetic, one rounding to E); the fp8 codes encode that value with the copy's
// own absmax.
template <typename E, int XM>
__device__ inline void copy_xform(Vec8<E>& x, const AppendArgs& a, const TileUnit& u, int row, int col) {
  if constexpr (XM > 0) {
    Vec8<float> y = to_f32(x);
    const float* m = XM == 2 ? a.kv_xf + ((int64_t)u.f * a.B + u.b) * 16 : nullptr;
    if (!u.is_v) {
      rope_spatial8(y, col, u.t * kTile + row, a.gh, a.gw, a.rope_hw);
      if constexpr (XM == 2) {
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
          if (col + 4 * gg >= 2 * kRopeT) xform4(y, gg, m);
      }
    } else if constexpr (XM == 2) {
      xform4(y, 0, m);
      xform4(y, 1, m);
    }
    x = from_f32<E>(y);
  }
}

template <typename E>
__device__ inline const E* tile_src(const AppendArgs& a, const TileUnit& u) {
  return static_cast<const E*>(u.is_v ? a.vsrc : a.ksrc) + (int64_t)u.b * a.s_sb +
         (int64_t)u.h * a.s_sh + ((int64_t)(a.src_frame0 + u.f) * a.T + u.t * kTile) * a.s_st;
}

template <typename E, int XM = 0>
__global__ __launch_bounds__(256) void fp8_tile_absmax_kernel(AppendArgs a, float* part) {
  __shared__ float red[4];
  const TileUnit u(a, XM == 1);
  const E* src = tile_src<E>(a, u);
  const int tid = threadIdx.x, rows = min(kTile, a.T - u.t * kTile);
  const bool knorm = !u.is_v && a.krms;
  const int64_t tok0 = (int64_t)(a.src_frame0 + u.f) * a.T + u.t * kTile;
  float m = 0.f;
  // 64 rows x 16 vec8 = 4 per thread, all loads issued first (rows past T read the last valid
  // row and are skipped below); plain loads, so the second pass can find the tile in L2/MALL
  Vec8<E> x[4];
  const int col = (tid & 15) * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    x[i] = Vec8<E>::load(src + (int64_t)min((tid >> 4) + 16 * i, rows - 1) * a.s_st + col);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (tid >> 4) + 16 * i;
    if (row < rows) {
      if (knorm) norm8(x[i], a, u.b, u.h, tok0 + row, col);
      copy_xform<E, XM>(x[i], a, u, row, col);
      m = absval8(x[i], m);
    }
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <typename E>
__device__ inline u32x2 quant_vec8(const Vec8<E>& v, float inv);
template <>
__device__ inline u32x2 quant_vec8<bf16>(const Vec8<bf16>& v, float inv) {
  return quant8(v.r, inv);
}
template <>
__device__ inline u32x2 quant_vec8<float>(const Vec8<float>& v, float inv) {
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t code = f32_to_e4m3(fminf(fmaxf(v.get(i) * inv, -448.0f), 448.0f));
    if (i < 4) lo |= code << (8 * i); else hi |= code << (8 * (i - 4));
  }
  return u32x2{lo, hi};
}

template <typename E, int XM = 0>
__global__ __launch_bounds__(256) void append_fp8_tile_kernel(AppendArgs a, const float* part) {
  constexpr int kRowT = kTile + 4;  // V^T tile row: 64 codes + 4 bytes of skew
  __shared__ __attribute__((aligned(16))) uint8_t vt8[kHeadDim * kRowT];
  const TileUnit u(a, XM == 1);
  const E* src = tile_src<E>(a, u);
  const int tid = threadIdx.x, rows = min(kTile, a.T - u.t * kTile);
  const float* pm = part + (int64_t)(blockIdx.x - u.t);
  float amax = 0.f;
  for (int i = 0; i < a.ntiles; ++i) amax = fmaxf(amax, pm[i]);
  const float inv = amax > 0.f ? 448.0f / amax : 0.f;
  const int64_t slot = a.slots[u.f];
  if (u.t == 0 && tid == 0) {
    float* sc = XM ? (u.is_v ? a.vrscale : a.krscale) : (u.is_v ? a.vscale : a.kscale);
    sc[(slot * a.B + u.b) * a.H + u.h] = amax / 448.0f;
  }
  const bool knorm = !u.is_v && a.krms;
  const int64_t tok0 = (int64_t)(a.src_frame0 + u.f) * a.T + u.t * kTile;
  void* dst_pool = XM ? (u.is_v ? a.vrpool : a.krpool) : (u.is_v ? a.vpool : a.kpool);
  uint8_t* pool = static_cast<uint8_t*>(dst_pool) + slot * a.slot_stride +
                  (int64_t)(u.b * a.H + u.h) * a.Tp * kHeadDim;
  u32x2 q[4];
  Vec8<E> x[4];
  {
    const int col = (tid & 15) * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i)  // all loads first; rows past T become code 0 below
      x[i] = Vec8<E>::load_nt(src + (int64_t)min((tid >> 4) + 16 * i, rows - 1) * a.s_st + col);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (tid >> 4) + 16 * i;
      if (row >= rows) {
        x[i] = Vec8<E>::zero();
      } else {
        if (knorm) norm8(x[i], a, u.b, u.h, tok0 + row, col);
        copy_xform<E, XM>(x[i], a, u, row, col);
      }
      q[i] = quant_vec8<E>(x[i], inv);
    }
  }
  if (!u.is_v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 4, col = (c & 15) * 8;
      *reinterpret_cast<u32x2*>(pool + (int64_t)(u.t * kTile + row) * kHeadDim + col) = q[i];
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + 256 * i, row = c >> 4, col = (c & 15) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) vt8[(col + e) * kRowT + row] = (uint8_t)(q[i][e >> 2] >> (8 * (e & 3)));
  }
  __syncthreads();
  // channel d, tokens tc .. tc+31 of the tile
  const int d = tid >> 1, tc = (tid & 1) * 32;
  const uint32_t* rd = reinterpret_cast<const uint32_t*>(vt8 + d * kRowT + tc);
  uint8_t* dst = pool + (int64_t)d * a.Tp + u.t * kTile + tc;
  st_nt(dst, u32x4{rd[0], rd[1], rd[2], rd[3]});
  st_nt(dst + 16, u32x4{rd[4], rd[5], rd[6], rd[7]});
}

// fp8 append in one pass for chunks with few (frame, batch, head, K|V) units (fewer than 4 per
// CU, e.g. C5: 288 units of 25 tiles on 256 CUs).  Each unit is cut into slices of at most
// kSliceTiles 64-token tiles, one 256-thread workgroup per slice, and the grid is no larger
// than the chip holds at once (occupancy x CUs), so every slice is resident: together the slices
// hold the whole chunk on chip (C5: 115 MB of bf16 K/V in 2016 workgroups of 64 KB, against
// 168 MB of registers and LDS) and HBM is read once.  A workgroup issues all of its slice's loads at once (12 vectors
// per thread into registers, 4 into LDS by direct buffer loads), reduces the slice absmax,
// publishes it in its own word of the unit's cell (one 64-bit device-scope atomic store of
// (1 << 32) | absmax bits: the value and its presence travel together, so no other memory
// ordering is needed), waits until every slice of the unit has published (one lane per slice
// polls) and encodes with the unit's absmax: the frame absmax the per-unit kernels reduce, so
// codes and scales are bit-identical to theirs.
//   K: thread t owns the 16 B vectors at row (t >> 4) + 16 i of each tile, channels
//      (t & 15) * 8 .. +8 (four rows of 256 B per wave instruction); codes are 8 B per vector.
//   V: thread t owns two 8-token x 8-channel blocks, tokens 128 k + 8 (t & 15) .. +8 of the
//      slice, channels 8 (t >> 4) .. +8.  Codes are packed channel-major (each e4m3 pack takes
//      one channel of successive tokens), so a store writes one channel's 8 token codes and 16
//      lanes fill a 128 B line of V^T: no transpose buffer, no partial lines.
// Residency is what the grid size aims for, not what the launch guarantees (other work may hold
// CUs), so no result depends on it: the wait is bounded in time (wait_ticks of the 100 MHz
// real-time counter), and a workgroup whose unit has not completed by then reads the whole
// unit again to form the same absmax itself (correct, slower; word 0 of the workspace then
// records that a fallback ran).  fp8_slice_clear_kernel zeroes the cells just before, on the
// same stream, so the workspace keeps no state between calls.
constexpr int kSliceTiles = 4;
constexpr int kSliceRegVecs = 12;  // of the 16 vectors a thread owns; the other 4 go to LDS
constexpr int kSliceMax = 64;      // slices per unit (one polling lane each)
constexpr int kSliceHead = 16;     // workspace words before the first cell (128 B)

struct SliceSync {
  unsigned long long* cells;  // word 0: fallback flag; unit u's cell at kSliceHead + u * cell_words
  int slices;                 // slices per unit, <= kSliceMax
  int tps;                    // tiles per slice, <= kSliceTiles
  int cell_words;             // slices rounded up to 16 (whole 128 B lines per unit)
  unsigned int wait_ticks;    // bound of the wait for the unit's other slices
};

__global__ __launch_bounds__(256) void fp8_slice_clear_kernel(unsigned long long* cells, int n_words) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n_words; i += gridDim.x * 256) cells[i] = 0ull;
}

__device__ inline float e4m3_in(uint32_t w, bool hi, float inv) {
  const float x = __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
  return fminf(fmaxf(x * inv, -448.0f), 448.0f);
}

// One slice (K when !V, V^T when V): load, reduce, publish, wait, encode.
template <bool V>
__device__ __forceinline__ void fp8_slice(const AppendArgs& a, const SliceSync& sy, int unit, int s,
                                          int h, int b, int f, uint8_t (*stage)[256 * 16], float* red) {
  const int t0 = s * sy.tps;
  const int nt = min(sy.tps, a.ntiles - t0);
  const int row0 = t0 * kTile;
  const int live = min(a.T - row0, nt * kTile);  // >= 1: t0 < ntiles = ceil(T / 64)
  const int tid = threadIdx.x;
  // lane part and uniform part of vector j's row within the slice
  const int lrow = V ? 8 * (tid & 15) : tid >> 4;
  const int lcol = V ? 8 * (tid >> 4) : 8 * (tid & 15);
  auto urow = [](int j) { return V ? 128 * (j >> 3) + (j & 7) : 64 * (j >> 2) + 16 * (j & 3); };
  const bf16* src = static_cast<const bf16*>(V ? a.vsrc : a.ksrc) + (int64_t)b * a.s_sb +
                    (int64_t)h * a.s_sh + ((int64_t)(a.src_frame0 + f) * a.T + row0) * a.s_st;
  // the host guarantees a slice spans < 2^31 bytes: one 32-bit lane offset per thread, the
  // row offsets of vector j are uniform (scalar offset of the buffer load)
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, 0x7fffffff, 0x00020000);
  const uint32_t lane_off = (uint32_t)(lrow * a.s_st + lcol) * 2u;
  const uint32_t rstep = (uint32_t)a.s_st * 2u;
#pragma unroll
  for (int c = 0; c < 16 - kSliceRegVecs; ++c) {
    const int j = kSliceRegVecs + c;
    if (lrow < live - urow(j))
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(&stage[c][0] + (tid >> 6) * 1024),
                                               16, lane_off, urow(j) * rstep, 0, 0);
  }
  u32x4 r[kSliceRegVecs];
#pragma unroll
  for (int j = 0; j < kSliceRegVecs; ++j) {
    r[j] = u32x4{0u, 0u, 0u, 0u};
    if (lrow < live - urow(j))
      r[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off, urow(j) * rstep, 0));
  }
  // vector j wherever it lives, zero for rows >= T.  The LDS reads are volatile:
  // each phase reads the staged vectors again rather than keep 16 more registers live.
  auto vec = [&](int j) -> u32x4 {
    if (j < kSliceRegVecs) return r[j];
    if (lrow >= live - urow(j)) return u32x4{0u, 0u, 0u, 0u};
    typedef __attribute__((address_space(3))) const volatile u32x4 lds_u32x4;
    const u32x4 x = *(lds_u32x4*)(__attribute__((address_space(3))) const uint8_t*)
                         &stage[j - kSliceRegVecs][tid * 16];
    return x;
  };
  u16x2 mm = {0, 0};
#pragma unroll
  for (int j = 0; j < kSliceRegVecs; ++j) mm = absmax8(r[j], mm);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS vectors have landed
#pragma unroll
  for (int j = kSliceRegVecs; j < 16; ++j) {  // one staged vector at a time
    mm = absmax8(vec(j), mm);
    asm volatile("" : "+v"(mm) : : "memory");
  }
  float m = __uint_as_float((uint32_t)(mm[0] > mm[1] ? mm[0] : mm[1]) << 16);
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid < 64) {  // wave 0: publish, then lane l < slices polls slice l's word
    unsigned long long* cell = sy.cells + kSliceHead + (int64_t)unit * sy.cell_words;
    if (tid == 0) {
      const float ms = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
      __hip_atomic_store(cell + s, (1ull << 32) | __float_as_uint(ms), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint64_t t_end = __builtin_amdgcn_s_memrealtime() + sy.wait_ticks;
    unsigned long long w = 0;
    bool have = tid >= sy.slices;
    bool late = false;
    for (;;) {
      if (!have) {
        w = __hip_atomic_load(cell + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        have = (w >> 32) != 0;
      }
      if (__all(have)) break;
      if (__builtin_amdgcn_s_memrealtime() >= t_end) {
        late = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    float um = __uint_as_float((uint32_t)w);  // 0 for lanes past the unit's slices
    for (int off = 32; off > 0; off >>= 1) um = fmaxf(um, __shfl_xor(um, off));
    if (tid == 0) red[4] = late ? -1.0f : um;
  }
  __syncthreads();
  if (red[4] < 0.f) {  // the unit did not complete in time (uniform branch): read all of it
    // (rows [0, T) of the frame), then load this slice's register vectors again, so they need
    // no registers while the whole-unit loop runs; the LDS vectors are still in place
    const bf16* fsrc = src - (int64_t)row0 * a.s_st;
    u16x2 fm = {0, 0};
    for (int c = tid; c < a.T * 16; c += 256)
      fm = absmax8(ld_nt(fsrc + (int64_t)(c >> 4) * a.s_st + (c & 15) * 8), fm);
    float x = __uint_as_float((uint32_t)(fm[0] > fm[1] ? fm[0] : fm[1]) << 16);
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    __syncthreads();  // every read of red[0..4] above is done
    if ((tid & 63) == 0) red[tid >> 6] = x;
    __syncthreads();
    if (tid == 0) {
      red[4] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
      __hip_atomic_store(sy.cells, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int j = 0; j < kSliceRegVecs; ++j) {
      r[j] = u32x4{0u, 0u, 0u, 0u};
      if (lrow < live - urow(j))
        r[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off, urow(j) * rstep, 0));
    }
    __syncthreads();
  }
  const float amax = red[4];
  const float inv = amax > 0.f ? 448.0f / amax : 0.f;
  const int64_t slot = a.slots[f];
  if (s == 0 && tid == 0) {
    float* sc = V ? a.vscale : a.kscale;
    sc[(slot * a.B + b) * a.H + h] = amax / 448.0f;
  }
  // codes go out through a buffer resource over the (slot, b, h) block (Tp x 128 bytes):
  // lane offset in one VGPR, the vector's uniform offset scalar, nontemporal (aux bit 1)
  uint8_t* pool = static_cast<uint8_t*>(V ? a.vpool : a.kpool) + slot * a.slot_stride +
                  (int64_t)(b * a.H + h) * a.Tp * kHeadDim;
  const __amdgpu_buffer_rsrc_t ps =
      __builtin_amdgcn_make_buffer_rsrc((void*)pool, (short)0, a.Tp * kHeadDim, 0x00020000);
  const int rows = nt * kTile;  // the slice's pool rows, padding (code 0) included
  if (!V) {
    const uint32_t st_lane = (uint32_t)((row0 + lrow) * kHeadDim + lcol);
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (lrow < rows - urow(j))
        __builtin_amdgcn_raw_buffer_store_b64(quant8(vec(j), inv), ps, st_lane, urow(j) * kHeadDim, 2);
    return;
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int tok = 128 * k + lrow;
    if (tok >= rows) continue;
    u32x4 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = vec(8 * k + i);
    const uint32_t st_lane = (uint32_t)(lcol * a.Tp + row0 + tok);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int w = c >> 1;
      const bool hi = c & 1;
      const u32x2 q{e4m3x4(e4m3_in(x[0][w], hi, inv), e4m3_in(x[1][w], hi, inv),
                           e4m3_in(x[2][w], hi, inv), e4m3_in(x[3][w], hi, inv)),
                    e4m3x4(e4m3_in(x[4][w], hi, inv), e4m3_in(x[5][w], hi, inv),
                           e4m3_in(x[6][w], hi, inv), e4m3_in(x[7][w], hi, inv))};
      __builtin_amdgcn_raw_buffer_store_b64(q, ps, st_lane, c * a.Tp, 2);
    }
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8)))
void append_fp8_slice_kernel(AppendArgs a, SliceSync sy) {
  __shared__ __attribute__((aligned(16))) uint8_t stage[16 - kSliceRegVecs][256 * 16];
  __shared__ float red[5];
  const int unit = blockIdx.x / sy.slices;
  const int s = blockIdx.x - unit * sy.slices;
  int wg = unit >> 1;
  const int h = wg % a.H;
  wg /= a.H;
  const int b = wg % a.B;
  const int f = wg / a.B;
  if (unit & 1)
    fp8_slice<true>(a, sy, unit, s, h, b, f, stage, red);
  else
    fp8_slice<false>(a, sy, unit, s, h, b, f, stage, red);
}

// Inverse RMS of each token's H x D row (WanRMSNorm's statistic, model.py:69-84):
// out[b * rows + t] = 1 / sqrt(mean(x^2) + eps) in fp32.  One wave per token: lane l sums the
// squares of 8-element chunks l, l+64, ... of the row (chunk c = head c / 16, channels
// (c % 16) * 8 .. +8), then the wave reduces.
struct RmsArgs {
  const void* x;
  int64_t sb, st, sh;
  int B, rows, H;
  float eps;
  float* out;
};

template <typename E>
__global__ __launch_bounds__(256) void rms_rows_kernel(RmsArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.B * a.rows) return;  // whole waves
  const int b = row / a.rows, t = row - b * a.rows;
  const int lane = threadIdx.x & 63;
  const E* base = static_cast<const E*>(a.x) + (int64_t)b * a.sb + (int64_t)t * a.st;
  float s = 0.f;
  for (int c = lane; c < a.H * 16; c += 64) {
    const Vec8<E> v = Vec8<E>::load(base + (int64_t)(c >> 4) * a.sh + (c & 15) * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = (float)v.get(e);
      s = fmaf(x, x, s);
    }
  }
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) a.out[row] = 1.0f / sqrtf(s / (float)(a.H * kHeadDim) + a.eps);
}

struct GatherArgs {
  const void* kpool;
  const void* vpool;
  void* kout;
  void* vout;
  int64_t o_sb, o_st, o_sh;
  int64_t slot_stride;
  int B, H, T, Tp, n_frames, ntiles;
  int32_t slots[SKV_MAX_FRAMES];
};

// grid.x = n_frames * B * H * ntiles, block = 256; E is the raw element type of the pool.
// Threads 0-127 copy the tile's K rows (16 B vectors); threads 128-255 each read an 8-channel x
// 8-token block of V^T and write it transposed (8 token rows of 8 channels), in registers.
template <typename E>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
  int wg = blockIdx.x;
  const int t = wg % a.ntiles;
  wg /= a.ntiles;
  const int h = wg % a.H;
  wg /= a.H;
  const int b = wg % a.B;
  const int f = wg / a.B;
  const int64_t slot = a.slots[f];
  const int tid = threadIdx.x;
  const int tok0 = t * kTile;
  const int64_t obase = (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)f * a.T * a.o_st;
  if (tid < 128) {
    const E* __restrict__ kp = static_cast<const E*>(a.kpool) + slot * a.slot_stride +
                               ((int64_t)(b * a.H + h) * a.Tp + tok0) * kHeadDim;
    E* __restrict__ ko = static_cast<E*>(a.kout) + obase;
    // all loads first, then the stores; padding rows re-read the frame's last row (same line,
    // no HBM traffic) and are not stored
    const int col = (tid & 15) * 8;
    const int last = a.T - 1 - tok0;
    Vec8<E> kv[8];
#pragma unroll
    for (int r = 0; r < 8; ++r)
      kv[r] = Vec8<E>::load_nt(kp + min((tid >> 4) + 8 * r, last) * kHeadDim + col);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int row = (tid >> 4) + 8 * r;
      if (tok0 + row < a.T) kv[r].store_nt(ko + (int64_t)(tok0 + row) * a.o_st + col);
    }
    return;
  }
  const E* __restrict__ vp = static_cast<const E*>(a.vpool) + slot * a.slot_stride +
                             (int64_t)(b * a.H + h) * kHeadDim * a.Tp + tok0;
  E* __restrict__ vo = static_cast<E*>(a.vout) + obase;
  const int i = tid - 128;
  const int tb = i & 7, db = i >> 3;  // tokens tb*8.., channels db*8..
  const int tokb = tok0 + tb * 8;
  // a vector of padding tokens only re-reads the frame's last vector (its values are not
  // stored): vectors that start at or past T cost no HBM traffic
  const int tcol = min(tokb, ((a.T - 1) >> 3) << 3) - tok0;
  if constexpr (sizeof(E) == 2) {
    u32x4 in[8], out[8];
#pragma unroll
    for (int r = 0; r < 8; ++r)
      in[r] = ld_nt(vp + (int64_t)(db * 8 + r) * a.Tp + tcol);
    transpose8x8_b16(in, out);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      if (tokb + c < a.T)
        st_nt(vo + (int64_t)(tokb + c) * a.o_st + db * 8, out[c]);
  } else {
    Vec8<E> in[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) in[r] = Vec8<E>::load_nt(vp + (int64_t)(db * 8 + r) * a.Tp + tcol);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      Vec8<E> o;
#pragma unroll
      for (int r = 0; r < 8; ++r) o.set(r, in[r].get(c));
      if (tokb + c < a.T) o.store_nt(vo + (int64_t)(tokb + c) * a.o_st + db * 8);
    }
  }
}

// fp8 pools hold raw bytes; gather copies the codes (scales stay in the scale arrays).
struct U8x8 {
  uint8_t b[8];
};

__global__ __launch_bounds__(256) void gather_u8_kernel(GatherArgs a) {
  __shared__ uint8_t vt[kHeadDim * (kTile + 16)];
  int wg = blockIdx.x;
  const int t = wg % a.ntiles;
  wg /= a.ntiles;
  const int h = wg % a.H;
  wg /= a.H;
  const int b = wg % a.B;
  const int f = wg / a.B;
  const int64_t slot = a.slots[f];
  const int tid = threadIdx.x;
  const int tok0 = t * kTile;
  constexpr int kRow = kTile + 16;
  const uint8_t* kp = static_cast<const uint8_t*>(a.kpool) + slot * a.slot_stride +
                      ((int64_t)(b * a.H + h) * a.Tp + tok0) * kHeadDim;
  const uint8_t* vp = static_cast<const uint8_t*>(a.vpool) + slot * a.slot_stride +
                      (int64_t)(b * a.H + h) * kHeadDim * a.Tp + tok0;
  uint8_t* ko = static_cast<uint8_t*>(a.kout) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
                (int64_t)f * a.T * a.o_st;
  uint8_t* vo = static_cast<uint8_t*>(a.vout) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
                (int64_t)f * a.T * a.o_st;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = tid + 256 * r;
    const int d = c >> 3, tc = (c & 7) * 8;
    u32x2 v = *reinterpret_cast<const u32x2*>(vp + (int64_t)d * a.Tp + tc);
    *reinterpret_cast<u32x2*>(vt + d * kRow + tc) = v;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = tid + 256 * r;
    const int row = c >> 4, col = (c & 15) * 8;
    if (tok0 + row < a.T) {
      const int64_t oo = (int64_t)(tok0 + row) * a.o_st + col;
      *reinterpret_cast<u32x2*>(ko + oo) = *reinterpret_cast<const u32x2*>(kp + row * kHeadDim + col);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t code = vt[(col + i) * kRow + row];
        if (i < 4) lo |= code << (8 * i); else hi |= code << (8 * (i - 4));
      }
      *reinterpret_cast<u32x2*>(vo + oo) = u32x2{lo, hi};
    }
  }
}

}  // namespace skv

using namespace skv;

// Tiles per slice of the one-pass fp8 append for `units` units of `ntiles` tiles: the fewest
// that let every slice be resident at once (workgroups of append_fp8_slice_kernel per CU, from
// the occupancy query, times the CUs), or 0 when more than kSliceTiles would be needed.
static int slice_tiles(int ntiles, int units) {
  static int per_cu = -1;
  if (per_cu < 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, (const void*)append_fp8_slice_kernel, 256, 0) !=
        hipSuccess) {
      (void)hipGetLastError();
      nb = 0;
    }
    per_cu = nb;
  }
  const int64_t resident = (int64_t)per_cu * cu_count();
  for (int tps = 1; tps <= kSliceTiles; ++tps) {
    const int slices = (ntiles + tps - 1) / tps;
    if (slices <= kSliceMax && (int64_t)units * slices <= resident) return tps;
  }
  return 0;
}

// Bound of the one-pass append's wait, in ticks of the 100 MHz real-time counter: 200 us (the
// whole C5 chunk loads in ~20 us), or SOLARKV_SLICE_WAIT_US, read on every call, so that tests
// can force the fallback from the host (0 = never wait).
static unsigned int slice_wait_ticks() {
  const char* e = getenv("SOLARKV_SLICE_WAIT_US");
  long us = 200;
  if (e && *e) {
    char* end = nullptr;
    const long v = strtol(e, &end, 10);
    if (end && *end == 0 && v >= 0 && v <= 10000000) us = v;
  }
  return (unsigned int)(us * 100);
}

static bool aligned8(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)(8 * bytes)) == 0; }

static int launch_status() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("skv_append: launch failed: %s", hipGetErrorString(e));
    return SKV_E_LAUNCH;
  }
  return SKV_OK;
}

// The fp8 copies of a pre-RoPE cache (after the raw frames): the tile grids' two passes over
// the K units (RoPE copy) or the K and V units (PRoPE copies), tile maxima in `part`.
static int append_fp8_copies(const AppendArgs& a, int src_dtype, int copy_units, void* part_ws,
                             hipStream_t s) {
  float* part = static_cast<float*>(part_ws);
  const dim3 grid(copy_units * a.ntiles), block(256);
  const bool prope = a.vrpool != nullptr;
  if (src_dtype == SKV_BF16) {
    if (prope) {
      hipLaunchKernelGGL((fp8_tile_absmax_kernel<bf16, 2>), grid, block, 0, s, a, part);
      hipLaunchKernelGGL((append_fp8_tile_kernel<bf16, 2>), grid, block, 0, s, a, part);
    } else {
      hipLaunchKernelGGL((fp8_tile_absmax_kernel<bf16, 1>), grid, block, 0, s, a, part);
      hipLaunchKernelGGL((append_fp8_tile_kernel<bf16, 1>), grid, block, 0, s, a, part);
    }
  } else {
    if (prope) {
      hipLaunchKernelGGL((fp8_tile_absmax_kernel<float, 2>), grid, block, 0, s, a, part);
      hipLaunchKernelGGL((append_fp8_tile_kernel<float, 2>), grid, block, 0, s, a, part);
    } else {
      hipLaunchKernelGGL((fp8_tile_absmax_kernel<float, 1>), grid, block, 0, s, a, part);
      hipLaunchKernelGGL((append_fp8_tile_kernel<float, 1>), grid, block, 0, s, a, part);
    }
  }
  return launch_status();
}

static int append_impl(const void* k_new, const void* v_new, int src_dtype, int64_t src_sb,
                       int64_t src_st, int64_t src_sh, int src_frame0, void* k_pool,
                       void* v_pool, float* k_scale, float* v_scale, int pool_dtype,
                       int n_slots, const int32_t* dst_slots, int n_frames, int batch,
                       int heads, int head_dim, int frame_tokens, void* kr_pool,
                       const float* rope_hw, int grid_h, int grid_w, void* vr_pool,
                       const float* kv_xform, skv_stream_t stream,
                       const float* k_inv_rms = nullptr, int64_t rms_sb = 0,
                       const float* k_norm_weight = nullptr, void* workspace = nullptr,
                       int64_t workspace_bytes = 0, int64_t* ws_query = nullptr,
                       float* kr_scale = nullptr, float* vr_scale = nullptr) {
  if (ws_query) *ws_query = 0;
  if (!k_new || !v_new || !k_pool || !v_pool || !dst_slots) {
    set_error("skv_append: null pointer argument");
    return SKV_E_ARG;
  }
  if (head_dim != kHeadDim) {
    set_error("skv_append: head_dim=%d unsupported (built for %d)", head_dim, kHeadDim);
    return SKV_E_UNSUPPORTED;
  }
  if (n_frames < 0 || n_frames > SKV_MAX_APPEND_FRAMES || batch <= 0 || heads <= 0 ||
      frame_tokens <= 0 || n_slots <= 0 || src_frame0 < 0) {
    set_error("skv_append: bad sizes (n_frames=%d batch=%d heads=%d T=%d n_slots=%d frame0=%d)",
              n_frames, batch, heads, frame_tokens, n_slots, src_frame0);
    return SKV_E_ARG;
  }
  if (workspace_bytes < 0 || (workspace == nullptr && workspace_bytes != 0)) {
    set_error("skv_append_ex: workspace_bytes=%lld without a workspace pointer",
              (long long)workspace_bytes);
    return SKV_E_ARG;
  }
  if (n_frames == 0) return SKV_OK;
  const bool fp8 = pool_dtype == SKV_FP8_E4M3;
  if (!(src_dtype == SKV_BF16 || src_dtype == SKV_F32 || src_dtype == SKV_F16) ||
      !(pool_dtype == src_dtype || (fp8 && src_dtype != SKV_F16))) {
    set_error("skv_append: src_dtype=%d pool_dtype=%d unsupported (pool must equal src or be fp8)",
              src_dtype, pool_dtype);
    return SKV_E_UNSUPPORTED;
  }
  // f16 chunks move bit for bit through the bf16 kernel (a plain append converts nothing); the
  // K norm and the RoPE / PRoPE copies compute, so they stay bf16 / f32 only
  if (src_dtype == SKV_F16 && (kr_pool || vr_pool || kv_xform || k_inv_rms)) {
    set_error("skv_append: f16 pools take plain appends only (no K norm, RoPE or PRoPE copies)");
    return SKV_E_UNSUPPORTED;
  }
  if (kr_pool) {
    if (fp8 && (!kr_scale || (vr_pool && !vr_scale))) {
      set_error("skv_append_ex: fp8 RoPE / PRoPE copies need kr_scale (and vx_scale with vx_pool)");
      return SKV_E_ARG;
    }
    if (!rope_hw || grid_h <= 0 || grid_w <= 0 || (int64_t)grid_h * grid_w != frame_tokens) {
      set_error("skv_append_rope: need rope_hw and grid_h * grid_w == frame_tokens (%d x %d vs %d)",
                grid_h, grid_w, frame_tokens);
      return SKV_E_ARG;
    }
  }
  if (vr_pool || kv_xform) {
    if (!vr_pool || !kv_xform || !kr_pool) {
      set_error("skv_append_prope: need kx_pool, vx_pool and kv_xform");
      return SKV_E_ARG;
    }
    if (pool_dtype != SKV_BF16 && !fp8) {
      set_error("skv_append_prope: only bf16 and fp8 pools are supported");
      return SKV_E_UNSUPPORTED;
    }
  }
  if (fp8 && (!k_scale || !v_scale)) {
    set_error("skv_append: fp8 pool needs k_scale and v_scale");
    return SKV_E_ARG;
  }
  if ((k_inv_rms == nullptr) != (k_norm_weight == nullptr)) {
    set_error("skv_append_ex: K RMSNorm needs both k_inv_rms and k_norm_weight");
    return SKV_E_ARG;
  }
  if (k_inv_rms && rms_sb < (int64_t)(src_frame0 + n_frames) * frame_tokens) {
    set_error("skv_append_ex: k_rms_stride_b=%lld is shorter than the source frames",
              (long long)rms_sb);
    return SKV_E_ARG;
  }
  const int esz = src_dtype == SKV_F32 ? 4 : 2;
  if (src_sb % 8 || src_st % 8 || src_sh % 8 || !aligned8(k_new, esz) || !aligned8(v_new, esz)) {
    set_error("skv_append: source strides/pointers must be multiples of 8 elements");
    return SKV_E_ARG;
  }
  AppendArgs a;
  a.ksrc = k_new;
  a.vsrc = v_new;
  a.s_sb = src_sb;
  a.s_st = src_st;
  a.s_sh = src_sh;
  a.kpool = k_pool;
  a.vpool = v_pool;
  a.kscale = k_scale;
  a.vscale = v_scale;
  a.B = batch;
  a.H = heads;
  a.T = frame_tokens;
  a.Tp = padded_tokens(frame_tokens);
  a.n_frames = n_frames;
  a.src_frame0 = src_frame0;
  a.ntiles = a.Tp / kTile;
  a.slot_stride = (int64_t)batch * heads * a.Tp * kHeadDim;
  a.krpool = kr_pool;
  a.rope_hw = rope_hw;
  a.gh = grid_h;
  a.gw = grid_w;
  a.vrpool = vr_pool;
  a.kv_xf = kv_xform;
  a.krms = k_inv_rms;
  a.krms_sb = rms_sb;
  a.kw = k_norm_weight;
  a.krscale = kr_scale;
  a.vrscale = vr_scale;
  for (int f = 0; f < n_frames; ++f) {
    if (dst_slots[f] < 0 || dst_slots[f] >= n_slots) {
      set_error("skv_append: dst_slots[%d]=%d outside [0, %d)", f, dst_slots[f], n_slots);
      return SKV_E_ARG;
    }
    a.slots[f] = dst_slots[f];
  }
  // fp8 chunks with too few (frame, batch, head, K|V) units to fill the chip split them: into
  // resident slices (one pass, the units' cells in the caller's workspace) when the slices fit
  // the chip at once, else into 64-token tiles (two passes, one float per tile).
  const int units = n_frames * batch * heads * 2;
  const bool few_units = fp8 && units < 4 * cu_count();
  const int64_t tile_bytes = few_units ? (int64_t)units * a.ntiles * (int64_t)sizeof(float) : 0;
  const int64_t cell_bytes = few_units ? (kSliceHead + (int64_t)units * kSliceMax) * 8 : 0;
  const int64_t ws_need = tile_bytes > cell_bytes ? tile_bytes : cell_bytes;
  // fp8 copies of a pre-RoPE cache run the tile grids after the raw frames, on the same stream,
  // with their tile maxima at the workspace's start (the raw append is done with it by then)
  const int copy_units = fp8 && kr_pool ? n_frames * batch * heads * (vr_pool ? 2 : 1) : 0;
  const int64_t copy_bytes = (int64_t)copy_units * a.ntiles * (int64_t)sizeof(float);
  if (ws_query) {
    *ws_query = ws_need > copy_bytes ? ws_need : copy_bytes;
    return SKV_OK;
  }
  if (copy_units > 0) {
    if (workspace == nullptr || workspace_bytes < copy_bytes) {
      set_error("skv_append_ex: fp8 RoPE / PRoPE copies need a workspace of %lld bytes "
                "(skv_append_workspace_size), got %lld", (long long)copy_bytes,
                (long long)workspace_bytes);
      return SKV_E_ARG;
    }
    if (reinterpret_cast<uintptr_t>(workspace) % 4) {
      set_error("skv_append_ex: workspace must be 4-byte aligned");
      return SKV_E_ARG;
    }
  }
  bool tile_split = false;
  if (ws_need > 0 && workspace != nullptr) {
    if (workspace_bytes < ws_need) {
      set_error("skv_append_ex: workspace of %lld bytes is smaller than the %lld this fp8 append "
                "needs (skv_append_workspace_size)", (long long)workspace_bytes,
                (long long)ws_need);
      return SKV_E_ARG;
    }
    if (reinterpret_cast<uintptr_t>(workspace) % 4) {
      set_error("skv_append_ex: workspace must be 4-byte aligned");
      return SKV_E_ARG;
    }
    tile_split = true;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fp8) {
    // the one-pass kernel: bf16 sources without the K norm, token rows at least a head apart,
    // a slice spanning < 2^31 bytes, 8-byte aligned cells (else the tile grids below)
    if (tile_split && src_dtype == SKV_BF16 && !k_inv_rms && src_st >= kHeadDim &&
        (int64_t)kSliceTiles * kTile * src_st * 2 < ((int64_t)1 << 31) &&
        reinterpret_cast<uintptr_t>(workspace) % 8 == 0) {
      SliceSync sy;
      sy.cells = static_cast<unsigned long long*>(workspace);
      sy.tps = slice_tiles(a.ntiles, units);
      sy.slices = sy.tps > 0 ? (a.ntiles + sy.tps - 1) / sy.tps : 0;
      sy.cell_words = (sy.slices + 15) / 16 * 16;
      sy.wait_ticks = slice_wait_ticks();
      if (sy.tps > 0) {
        const int n_words = kSliceHead + units * sy.cell_words;
        hipLaunchKernelGGL(fp8_slice_clear_kernel, dim3((n_words + 255) / 256), dim3(256), 0, s,
                           sy.cells, n_words);
        hipLaunchKernelGGL(append_fp8_slice_kernel, dim3(units * sy.slices), dim3(256), 0, s, a, sy);
        return copy_units ? append_fp8_copies(a, src_dtype, copy_units, workspace, s) : launch_status();
      }
    }
    if (tile_split) {
      float* part = static_cast<float*>(workspace);
      dim3 tgrid(units * a.ntiles);
      if (src_dtype == SKV_BF16) {
        hipLaunchKernelGGL(fp8_tile_absmax_kernel<bf16>, tgrid, dim3(256), 0, s, a, part);
        hipLaunchKernelGGL(append_fp8_tile_kernel<bf16>, tgrid, dim3(256), 0, s, a, part);
      } else {
        hipLaunchKernelGGL(fp8_tile_absmax_kernel<float>, tgrid, dim3(256), 0, s, a, part);
        hipLaunchKernelGGL(append_fp8_tile_kernel<float>, tgrid, dim3(256), 0, s, a, part);
      }
    } else {
      dim3 grid(units);
      const bool reg_path = src_dtype == SKV_BF16 && a.ntiles <= kFp8OnChip &&
                            (int64_t)a.Tp * src_st * 2 < ((int64_t)1 << 31);
      if (reg_path)
        hipLaunchKernelGGL(append_fp8_reg_kernel, grid, dim3(1024), 0, s, a);
      else if (src_dtype == SKV_BF16)
        hipLaunchKernelGGL(append_fp8_kernel<bf16>, grid, dim3(1024), 0, s, a);
      else
        hipLaunchKernelGGL(append_fp8_kernel<float>, grid, dim3(1024), 0, s, a);
    }
    if (copy_units) return append_fp8_copies(a, src_dtype, copy_units, workspace, s);
  } else {
    dim3 grid(n_frames * batch * heads * a.ntiles);
    if (src_dtype == SKV_BF16 || src_dtype == SKV_F16) {
      if (kv_xform)
        hipLaunchKernelGGL((append_kernel<bf16, 2>), grid, dim3(256), 0, s, a);
      else if (kr_pool)
        hipLaunchKernelGGL((append_kernel<bf16, 1>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((append_kernel<bf16, 0>), grid, dim3(256), 0, s, a);
    } else {
      if (kr_pool)
        hipLaunchKernelGGL((append_kernel<float, 1>), grid, dim3(256), 0, s, a);
      else
        hipLaunchKernelGGL((append_kernel<float, 0>), grid, dim3(256), 0, s, a);
    }
  }
  return launch_status();
}

extern "C" int skv_append(const void* k_new, const void* v_new, int src_dtype, int64_t src_sb,
                          int64_t src_st, int64_t src_sh, int src_frame0, void* k_pool,
                          void* v_pool, float* k_scale, float* v_scale, int pool_dtype,
                          int n_slots, const int32_t* dst_slots, int n_frames, int batch,
                          int heads, int head_dim, int frame_tokens, skv_stream_t stream) {
  clear_error();
  return append_impl(k_new, v_new, src_dtype, src_sb, src_st, src_sh, src_frame0, k_pool, v_pool,
                     k_scale, v_scale, pool_dtype, n_slots, dst_slots, n_frames, batch, heads,
                     head_dim, frame_tokens, nullptr, nullptr, 0, 0, nullptr, nullptr, stream);
}

extern "C" int skv_append_rope(const void* k_new, const void* v_new, int src_dtype,
                               int64_t src_sb, int64_t src_st, int64_t src_sh, int src_frame0,
                               void* k_pool, void* v_pool, int pool_dtype, int n_slots,
                               const int32_t* dst_slots, int n_frames, int batch, int heads,
                               int head_dim, int frame_tokens, void* kr_pool,
                               const float* rope_hw, int grid_h, int grid_w,
                               skv_stream_t stream) {
  clear_error();
  if (!kr_pool) {
    set_error("skv_append_rope: null kr_pool");
    return SKV_E_ARG;
  }
  return append_impl(k_new, v_new, src_dtype, src_sb, src_st, src_sh, src_frame0, k_pool, v_pool,
                     nullptr, nullptr, pool_dtype, n_slots, dst_slots, n_frames, batch, heads,
                     head_dim, frame_tokens, kr_pool, rope_hw, grid_h, grid_w, nullptr, nullptr,
                     stream);
}

extern "C" int skv_append_prope(const void* k_new, const void* v_new, int src_dtype,
                                int64_t src_sb, int64_t src_st, int64_t src_sh, int src_frame0,
                                void* k_pool, void* v_pool, int pool_dtype, int n_slots,
                                const int32_t* dst_slots, int n_frames, int batch, int heads,
                                int head_dim, int frame_tokens, void* kx_pool, void* vx_pool,
                                const float* rope_hw, int grid_h, int grid_w,
                                const float* kv_xform, skv_stream_t stream) {
  clear_error();
  if (!kx_pool || !vx_pool || !kv_xform) {
    set_error("skv_append_prope: null kx_pool, vx_pool or kv_xform");
    return SKV_E_ARG;
  }
  return append_impl(k_new, v_new, src_dtype, src_sb, src_st, src_sh, src_frame0, k_pool, v_pool,
                     nullptr, nullptr, pool_dtype, n_slots, dst_slots, n_frames, batch, heads,
                     head_dim, frame_tokens, kx_pool, rope_hw, grid_h, grid_w, vx_pool, kv_xform,
                     stream);
}

static int append_desc(const skv_append_desc* d, skv_stream_t stream, int64_t* ws_query) {
  clear_error();
  if (!d) {
    set_error("skv_append_ex: null descriptor");
    return SKV_E_ARG;
  }
  if (d->kr_pool == nullptr && (d->vx_pool || d->kv_xform)) {
    set_error("skv_append_ex: PRoPE copies need kr_pool");
    return SKV_E_ARG;
  }
  return append_impl(d->k_new, d->v_new, d->src_dtype, d->src_sb, d->src_st, d->src_sh,
                     d->src_frame0, d->k_pool, d->v_pool, d->k_scale, d->v_scale, d->pool_dtype,
                     d->n_slots, d->dst_slots, d->n_frames, d->batch, d->heads, d->head_dim,
                     d->frame_tokens, d->kr_pool, d->rope_hw, d->grid_h, d->grid_w, d->vx_pool,
                     d->kv_xform, stream, d->k_inv_rms, d->k_rms_stride_b, d->k_norm_weight,
                     d->workspace, d->workspace_bytes, ws_query, d->kr_scale, d->vx_scale);
}

extern "C" int skv_append_ex(const skv_append_desc* d, skv_stream_t stream) {
  return append_desc(d, stream, nullptr);
}

extern "C" int skv_append_workspace_size(const skv_append_desc* d, int64_t* bytes) {
  if (!bytes) {
    clear_error();
    set_error("skv_append_workspace_size: null bytes");
    return SKV_E_ARG;
  }
  return append_desc(d, nullptr, bytes);
}

extern "C" int skv_rms_rows(const void* x, int dtype, int64_t sb, int64_t st, int64_t sh,
                            int batch, int rows, int heads, int head_dim, float eps,
                            float* inv_rms, skv_stream_t stream) {
  clear_error();
  if (!x || !inv_rms) {
    set_error("skv_rms_rows: null pointer argument");
    return SKV_E_ARG;
  }
  if (head_dim != kHeadDim) {
    set_error("skv_rms_rows: head_dim=%d unsupported (built for %d)", head_dim, kHeadDim);
    return SKV_E_UNSUPPORTED;
  }
  if (batch <= 0 || rows < 0 || heads <= 0 || !(eps >= 0.f)) {
    set_error("skv_rms_rows: bad sizes (batch=%d rows=%d heads=%d eps=%g)", batch, rows, heads,
              (double)eps);
    return SKV_E_ARG;
  }
  if (!(dtype == SKV_BF16 || dtype == SKV_F32)) {
    set_error("skv_rms_rows: dtype=%d unsupported", dtype);
    return SKV_E_UNSUPPORTED;
  }
  const int esz = dtype == SKV_F32 ? 4 : 2;
  if (sb % 8 || st % 8 || sh % 8 || !aligned8(x, esz)) {
    set_error("skv_rms_rows: strides/pointer must be multiples of 8 elements");
    return SKV_E_ARG;
  }
  if (rows == 0) return SKV_OK;
  RmsArgs a{x, sb, st, sh, batch, rows, heads, eps, inv_rms};
  const int64_t n = (int64_t)batch * rows;
  dim3 grid((unsigned)((n + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SKV_BF16)
    hipLaunchKernelGGL(rms_rows_kernel<bf16>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(rms_rows_kernel<float>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("skv_rms_rows: launch failed: %s", hipGetErrorString(e));
    return SKV_E_LAUNCH;
  }
  return SKV_OK;
}

extern "C" int skv_gather(const void* k_pool, const void* v_pool, int pool_dtype, int n_slots,
                          const int32_t* slots, int n_frames, int batch, int heads, int head_dim,
                          int frame_tokens, void* k_out, void* v_out, int64_t out_sb,
                          int64_t out_st, int64_t out_sh, skv_stream_t stream) {
  clear_error();
  if (!k_pool || !v_pool || !slots || !k_out || !v_out) {
    set_error("skv_gather: null pointer argument");
    return SKV_E_ARG;
  }
  if (head_dim != kHeadDim) {
    set_error("skv_gather: head_dim=%d unsupported (built for %d)", head_dim, kHeadDim);
    return SKV_E_UNSUPPORTED;
  }
  if (n_frames < 0 || n_frames > SKV_MAX_FRAMES || batch <= 0 || heads <= 0 ||
      frame_tokens <= 0 || n_slots <= 0) {
    set_error("skv_gather: bad sizes (n_frames=%d batch=%d heads=%d T=%d n_slots=%d)", n_frames,
              batch, heads, frame_tokens, n_slots);
    return SKV_E_ARG;
  }
  if (n_frames == 0) return SKV_OK;
  if (!(pool_dtype == SKV_BF16 || pool_dtype == SKV_F32 || pool_dtype == SKV_FP8_E4M3 ||
        pool_dtype == SKV_F16)) {
    set_error("skv_gather: pool_dtype=%d unsupported", pool_dtype);
    return SKV_E_UNSUPPORTED;
  }
  const int esz = pool_dtype == SKV_F32 ? 4 : (pool_dtype == SKV_FP8_E4M3 ? 1 : 2);
  if (out_sb % 8 || out_st % 8 || out_sh % 8 || !aligned8(k_out, esz) || !aligned8(v_out, esz)) {
    set_error("skv_gather: output strides/pointers must be multiples of 8 elements");
    return SKV_E_ARG;
  }
  GatherArgs a;
  a.kpool = k_pool;
  a.vpool = v_pool;
  a.kout = k_out;
  a.vout = v_out;
  a.o_sb = out_sb;
  a.o_st = out_st;
  a.o_sh = out_sh;
  a.B = batch;
  a.H = heads;
  a.T = frame_tokens;
  a.Tp = padded_tokens(frame_tokens);
  a.n_frames = n_frames;
  a.ntiles = a.Tp / kTile;
  a.slot_stride = (int64_t)batch * heads * a.Tp * kHeadDim;
  for (int f = 0; f < n_frames; ++f) {
    if (slots[f] < 0 || slots[f] >= n_slots) {
      set_error("skv_gather: slots[%d]=%d outside [0, %d)", f, slots[f], n_slots);
      return SKV_E_ARG;
    }
    a.slots[f] = slots[f];
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(n_frames * batch * heads * a.ntiles);
  if (pool_dtype == SKV_BF16 || pool_dtype == SKV_F16)  // 16-bit codes move bit for bit
    hipLaunchKernelGGL(gather_kernel<bf16>, grid, dim3(256), 0, s, a);
  else if (pool_dtype == SKV_F32)
    hipLaunchKernelGGL(gather_kernel<float>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(gather_u8_kernel, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("skv_gather: launch failed: %s", hipGetErrorString(e));
    return SKV_E_LAUNCH;
  }
  return SKV_OK;
}
