// Flash-style attention over a frame-slot KV pool for gfx950 (CDNA4).
//
// Replaces, for the cached Wan path, `attention(q, cat[sink, local])`
// (solar/backends/wan22/runtime/modeling/causal_model.py:1135-1226 -> attention.py:141-188)
// and, with mask_mode CHUNK_CAUSAL, the chunk-causal FlexAttention of causal_model.py:474-534.
// The key sequence is the concatenation of whole frames listed in a slot table, so the
// sink|local concatenation, the eviction memmove and the memory-bank gather of the reference
// all become addressing: nothing is copied before attention.
//
// Work decomposition (one workgroup = 4 waves = 128 queries of one (batch, head)):
//   * each wave owns 32 queries and keeps them in registers as the B operand of
//     v_mfma_f32_32x32x16_bf16, computing S^T = K Q^T so that one lane holds one query's
//     scores; the softmax row statistics then need a single cross-lane exchange (lane ^ 32);
//   * K (64 x 128) and V^T (128 x 64) tiles are staged in LDS and shared by the 4 waves;
//     the next tile's global loads are in flight while the current tile is computed;
//   * the K rows of each 32-key block are loaded in the permuted order key_perm(), which makes
//     the fp32 S^T accumulator of a lane hold, per 8 registers, 8 consecutive keys — exactly
//     the bf16x8 B operand (P^T) of the PV product; V is stored transposed in the pool so
//     its A operand (V^T rows) is one 16 B LDS read;
//   * tiles never straddle frames (frames are padded to 64 tokens); padding keys and keys
//     beyond a query's chunk-causal limit get -inf, decided per tile: full tiles skip the
//     mask, tiles past every query's limit are not visited.
#include <math.h>

#include "skv_common.h"

namespace skv {

struct AttnArgs {
  const void* q;
  void* o;
  const void* kpool;
  const void* vpool;
  const float* kscale;
  const float* vscale;
  int64_t q_sb, q_st, q_sh;
  int64_t o_sb, o_st, o_sh;
  int64_t slot_stride;
  int B, H, Lq, T, Tp, n_frames, ntiles_f, n_qtiles, n_wg;
  float scale_log2;  // softmax_scale * log2(e)
  int mask_mode;
  int64_t q_pos0, chunk, n_keys;
  int32_t slots[SKV_MAX_FRAMES];
};

constexpr int kBQ = 128;  // queries per workgroup (4 waves x 32)

// LDS holds each tile in MFMA operand order: one 1 KB block per A operand (64 lanes x 16 B),
// lane L of the block at byte L*16.  K tile: 16 blocks (kb, s) = 32-key block x 16-channel
// step; V^T tile: 16 blocks (db, kb, s2) = 32-channel block x 32-key block x 16-key step.
// A direct global->LDS load (global_load_lds_dwordx4) writes exactly one block, so staging
// needs no registers and every operand read is a linear, bank-conflict-free ds_read_b128.
constexpr int kBlockBytes = 1024;
constexpr int kTileBytes = 32 * kBlockBytes;  // K (16 KB) + V^T (16 KB)

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// Row m of a 32-row MFMA block reads key key_perm(m) of the block.  With the 32x32 C layout
// (lane l, register i -> row (i/4)*8 + (l/32)*4 + i%4) this puts key (i/8)*16 + (l/32)*8 + i%8
// in register i of lane l: each 8 registers are 8 consecutive keys, the B operand of PV.
__device__ inline int key_perm(int m) {
  const int a = m >> 3, h = (m >> 2) & 1, c = m & 3;
  return (a >> 1) * 16 + h * 8 + (a & 1) * 4 + c;
}

__device__ inline int64_t chunk_limit(int64_t pos, int64_t chunk, int64_t n_keys) {
  const int64_t lim = (pos / chunk + 1) * chunk;
  return lim < n_keys ? lim : n_keys;
}

template <typename OT>
__device__ inline void store4(OT* p, float x0, float x1, float x2, float x3);

template <>
__device__ inline void store4<bf16>(bf16* p, float x0, float x1, float x2, float x3) {
  bf16x4 v;
  v[0] = (bf16)x0; v[1] = (bf16)x1; v[2] = (bf16)x2; v[3] = (bf16)x3;
  *reinterpret_cast<bf16x4*>(p) = v;
}

template <>
__device__ inline void store4<float>(float* p, float x0, float x1, float x2, float x3) {
  *reinterpret_cast<f32x4*>(p) = f32x4{x0, x1, x2, x3};
}

// Stage tile `tau` into LDS buffer `buf`.  bf16 pools: 8 direct 16 B global->LDS loads per
// lane (4 K blocks + 4 V^T blocks per wave).  fp32 pools: loaded through registers and
// rounded to bf16 (the C1 fp32 path; not performance critical).
template <typename KT>
struct TileLoader;

template <>
struct TileLoader<bf16> {
  int64_t koff, voff;
  __device__ void init(int w, int lane, int Tp) {
    const int n = lane & 31, hh = lane >> 5;
    // wave w stages K blocks (kb = w>>1, s = (w&1)*4 + j) and V^T blocks (db = w, j = kb*2+s2)
    koff = (int64_t)((w >> 1) * 32 + key_perm(n)) * kHeadDim + (w & 1) * 64 + hh * 8;
    voff = (int64_t)(w * 32 + n) * Tp + hh * 8;
  }
  __device__ void issue(const bf16* kt, const bf16* vt, char* lds, int w) const {
    char* kdst = lds + (w * 4) * kBlockBytes;
    char* vdst = lds + 16 * kBlockBytes + (w * 4) * kBlockBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds((glb_void_t*)(kt + koff + j * 16),
                                       (lds_void_t*)(kdst + j * kBlockBytes), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds((glb_void_t*)(vt + voff + j * 16),
                                       (lds_void_t*)(vdst + j * kBlockBytes), 16, 0, 0);
  }
};

template <>
struct TileLoader<float> {
  int64_t koff, voff;
  int lane;
  __device__ void init(int w, int lane_, int Tp) {
    lane = lane_;
    const int n = lane & 31, hh = lane >> 5;
    koff = (int64_t)((w >> 1) * 32 + key_perm(n)) * kHeadDim + (w & 1) * 64 + hh * 8;
    voff = (int64_t)(w * 32 + n) * Tp + hh * 8;
  }
  __device__ void issue(const float* kt, const float* vt, char* lds, int w) const {
    char* kdst = lds + (w * 4) * kBlockBytes + lane * 16;
    char* vdst = lds + 16 * kBlockBytes + (w * 4) * kBlockBytes + lane * 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<bf16x8*>(kdst + j * kBlockBytes) = Vec8<float>::load(kt + koff + j * 16).to_bf16();
      *reinterpret_cast<bf16x8*>(vdst + j * kBlockBytes) = Vec8<float>::load(vt + voff + j * 16).to_bf16();
    }
  }
};

template <typename QT, typename KT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];  // 2 x kTileBytes

  // XCD-aware order: workgroup ids are dealt round-robin over the 8 XCDs; XCD x gets the
  // contiguous logical range starting at x*per + min(x, rem), so q-tiles of one head run on
  // one XCD and stream the same K/V through its L2.
  int logical;
  {
    const int bid = blockIdx.x, xcd = bid & 7, idx = bid >> 3;
    const int per = a.n_wg >> 3, rem = a.n_wg & 7;
    logical = xcd * per + min(xcd, rem) + idx;
  }
  const int qt = logical % a.n_qtiles;
  const int bh = logical / a.n_qtiles;
  const int h = bh % a.H, b = bh / a.H;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int q0 = qt * kBQ;
  const int qrow = q0 + w * 32 + n;
  const bool qlive = qrow < a.Lq;

  // Q^T operand: lane (n, hh) holds q[qrow][s*16 + hh*8 .. +7] for s = 0..7.
  bf16x8 qf[8];
  {
    const QT* qp = static_cast<const QT*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                   (int64_t)(qlive ? qrow : 0) * a.q_st + hh * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qf[s] = qlive ? Vec8<QT>::load(qp + s * 16).to_bf16() : Vec8<bf16>::zero().to_bf16();
  }

  // Visibility limits (keys are indexed 0..n_keys-1 in frame-list order).
  int64_t lim_lane = a.n_keys, lim_lo = a.n_keys, lim_hi = a.n_keys;
  if (a.mask_mode == SKV_MASK_CHUNK_CAUSAL) {
    const int qlast = min(q0 + kBQ, a.Lq) - 1;
    lim_lane = chunk_limit(a.q_pos0 + min(qrow, a.Lq - 1), a.chunk, a.n_keys);
    lim_lo = chunk_limit(a.q_pos0 + q0, a.chunk, a.n_keys);
    lim_hi = chunk_limit(a.q_pos0 + qlast, a.chunk, a.n_keys);
  }
  int ntau;
  {
    const int64_t jf = lim_hi / a.T;
    if (jf >= a.n_frames) {
      ntau = a.n_frames * a.ntiles_f;
    } else {
      const int64_t r = lim_hi - jf * a.T;
      ntau = (int)jf * a.ntiles_f + (int)((r + kTile - 1) / kTile);
    }
  }

  const KT* kpool = static_cast<const KT*>(a.kpool);
  const KT* vpool = static_cast<const KT*>(a.vpool);
  const int64_t kbh = (int64_t)(b * a.H + h) * a.Tp * kHeadDim;  // (b,h) offset inside a slot
  TileLoader<KT> loader;
  loader.init(w, lane, a.Tp);
  auto stage = [&](int tau, int buf) {
    const int j = tau / a.ntiles_f, t = tau - j * a.ntiles_f;
    const int64_t base = (int64_t)a.slots[j] * a.slot_stride + kbh;
    loader.issue(kpool + base + (int64_t)t * kTile * kHeadDim, vpool + base + t * kTile,
                 lds + buf * kTileBytes, w);
  };

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;
  // Running max in the log2 domain.  It is raised only when a tile's max exceeds it by more
  // than kStale, so most tiles skip the O rescale; probabilities then stay <= 2^kStale, which
  // bf16 and the fp32 sums represent exactly as well as values <= 1.
  constexpr float kStale = 8.0f;
  float m_run = -INFINITY, l_run = 0.f;
  const float c2 = a.scale_log2;
  const int lane16 = lane * 16;

  if (ntau > 0) {
    stage(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  for (int tau = 0; tau < ntau; ++tau) {
    const int buf = tau & 1;
    if (tau + 1 < ntau) stage(tau + 1, buf ^ 1);
    const char* kl = lds + buf * kTileBytes + lane16;
    const char* vl = kl + 16 * kBlockBytes;
    const int j = tau / a.ntiles_f, t = tau - j * a.ntiles_f;
    const int64_t key0 = (int64_t)j * a.T + t * kTile;
    const int tok0 = t * kTile;

    // S^T (64 keys x 32 queries per wave) = K Q^T
    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[kb][i] = 0.f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const bf16x8 ak = *reinterpret_cast<const bf16x8*>(kl + (kb * 8 + s) * kBlockBytes);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak, qf[s], sacc[kb], 0, 0, 0);
      }
    }

    const bool full = (tok0 + kTile <= a.T) && (key0 + kTile <= lim_lo);
    if (!full) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kk = kb * 32 + (i >> 3) * 16 + hh * 8 + (i & 7);
          if (tok0 + kk >= a.T || key0 + kk >= lim_lane) sacc[kb][i] = -INFINITY;
        }
    }

    // online softmax (base 2); lanes l and l^32 hold the two key halves of one query
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[kb][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * c2;
    if (mx > m_run + kStale) {
      // per lane: raise the reference point; the wave rescales only if some lane did
      const float alpha = __builtin_amdgcn_exp2f(m_run - mx);  // 0 when m_run == -inf
      m_run = mx;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;

    bf16x8 pb[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][i], c2, -m_use));
        l_run += p;
        pb[kb][i >> 3][i & 7] = (bf16)p;
      }

    // O^T (128 x 32 per wave) += V^T P^T
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8 av =
              *reinterpret_cast<const bf16x8*>(vl + (db * 4 + kb * 2 + s2) * kBlockBytes);
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb[kb][s2], oacc[db], 0, 0, 0);
        }

    // the next tile has landed in the other buffer; every wave is done with this one
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (qlive) {
    QT* op = static_cast<QT*>(a.o) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
             (int64_t)qrow * a.o_st;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + g * 8 + hh * 4;
        store4<QT>(op + d0, oacc[db][g * 4 + 0] * inv, oacc[db][g * 4 + 1] * inv,
                   oacc[db][g * 4 + 2] * inv, oacc[db][g * 4 + 3] * inv);
      }
  }
}

}  // namespace skv

using namespace skv;

extern "C" int skv_attention(const void* q, int q_dtype, int64_t q_sb, int64_t q_st,
                             int64_t q_sh, const void* k_pool, const void* v_pool,
                             const float* k_scale, const float* v_scale, int pool_dtype,
                             int n_slots, const int32_t* frame_slots, int n_frames, int batch,
                             int heads, int head_dim, int q_len, int frame_tokens,
                             float softmax_scale, int mask_mode, int64_t q_pos0,
                             int64_t chunk_tokens, void* out, int64_t out_sb, int64_t out_st,
                             int64_t out_sh, skv_stream_t stream) {
  clear_error();
  if (!q || !k_pool || !v_pool || !frame_slots || !out) {
    set_error("skv_attention: null pointer argument");
    return SKV_E_ARG;
  }
  if (head_dim != kHeadDim) {
    set_error("skv_attention: head_dim=%d unsupported (built for %d)", head_dim, kHeadDim);
    return SKV_E_UNSUPPORTED;
  }
  if (n_frames <= 0 || n_frames > SKV_MAX_FRAMES) {
    set_error("skv_attention: n_frames=%d outside [1, %d] (empty key window)", n_frames,
              SKV_MAX_FRAMES);
    return SKV_E_ARG;
  }
  if (batch <= 0 || heads <= 0 || q_len < 0 || frame_tokens <= 0 || n_slots <= 0) {
    set_error("skv_attention: bad sizes (batch=%d heads=%d Lq=%d T=%d n_slots=%d)", batch, heads,
              q_len, frame_tokens, n_slots);
    return SKV_E_ARG;
  }
  if (!(softmax_scale > 0.f)) {
    set_error("skv_attention: softmax_scale must be positive");
    return SKV_E_ARG;
  }
  if (mask_mode != SKV_MASK_NONE && mask_mode != SKV_MASK_CHUNK_CAUSAL) {
    set_error("skv_attention: unknown mask_mode %d", mask_mode);
    return SKV_E_ARG;
  }
  if (mask_mode == SKV_MASK_CHUNK_CAUSAL && (chunk_tokens <= 0 || q_pos0 < 0)) {
    set_error("skv_attention: chunk-causal mask needs chunk_tokens > 0 and q_pos0 >= 0");
    return SKV_E_ARG;
  }
  if (!(q_dtype == SKV_BF16 || q_dtype == SKV_F32)) {
    set_error("skv_attention: q_dtype=%d unsupported", q_dtype);
    return SKV_E_UNSUPPORTED;
  }
  if (!(pool_dtype == SKV_BF16 || pool_dtype == SKV_F32)) {
    set_error("skv_attention: pool_dtype=%d unsupported by this build", pool_dtype);
    return SKV_E_UNSUPPORTED;
  }
  if (q_sb % 8 || q_st % 8 || q_sh % 8 || out_sb % 4 || out_st % 4 || out_sh % 4) {
    set_error("skv_attention: q strides must be multiples of 8 and out strides of 4 elements");
    return SKV_E_ARG;
  }
  if (q_len == 0) return SKV_OK;
  AttnArgs a;
  a.q = q;
  a.o = out;
  a.kpool = k_pool;
  a.vpool = v_pool;
  a.kscale = k_scale;
  a.vscale = v_scale;
  a.q_sb = q_sb;
  a.q_st = q_st;
  a.q_sh = q_sh;
  a.o_sb = out_sb;
  a.o_st = out_st;
  a.o_sh = out_sh;
  a.B = batch;
  a.H = heads;
  a.Lq = q_len;
  a.T = frame_tokens;
  a.Tp = padded_tokens(frame_tokens);
  a.n_frames = n_frames;
  a.ntiles_f = a.Tp / kTile;
  a.n_qtiles = (q_len + kBQ - 1) / kBQ;
  a.n_wg = a.n_qtiles * heads * batch;
  a.slot_stride = (int64_t)batch * heads * a.Tp * kHeadDim;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.mask_mode = mask_mode;
  a.q_pos0 = q_pos0;
  a.chunk = chunk_tokens > 0 ? chunk_tokens : 1;
  a.n_keys = (int64_t)n_frames * frame_tokens;
  for (int j = 0; j < n_frames; ++j) {
    if (frame_slots[j] < 0 || frame_slots[j] >= n_slots) {
      set_error("skv_attention: frame_slots[%d]=%d outside [0, %d)", j, frame_slots[j], n_slots);
      return SKV_E_ARG;
    }
    a.slots[j] = frame_slots[j];
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(a.n_wg), block(256);
  const size_t lds_bytes = 2 * kTileBytes;
  if (q_dtype == SKV_BF16 && pool_dtype == SKV_BF16)
    hipLaunchKernelGGL((attn_kernel<bf16, bf16>), grid, block, lds_bytes, s, a);
  else if (q_dtype == SKV_BF16 && pool_dtype == SKV_F32)
    hipLaunchKernelGGL((attn_kernel<bf16, float>), grid, block, lds_bytes, s, a);
  else if (q_dtype == SKV_F32 && pool_dtype == SKV_BF16)
    hipLaunchKernelGGL((attn_kernel<float, bf16>), grid, block, lds_bytes, s, a);
  else
    hipLaunchKernelGGL((attn_kernel<float, float>), grid, block, lds_bytes, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("skv_attention: launch failed: %s", hipGetErrorString(e));
    return SKV_E_LAUNCH;
  }
  return SKV_OK;
}
