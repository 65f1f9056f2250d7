// Flash-style attention over a frame-slot KV pool for gfx950 (CDNA4).
//
// Replaces, for the cached Wan path, `attention(q, cat[sink, local])`
// (solar/backends/wan22/runtime/modeling/causal_model.py:1135-1226 -> attention.py:141-188)
// and, with mask_mode CHUNK_CAUSAL, the chunk-causal FlexAttention of causal_model.py:474-534.
// The key sequence is the concatenation of whole frames listed in a slot table, so the
// sink|local concatenation, the eviction memmove and the memory-bank gather of the reference
// all become addressing: nothing is copied before attention.
//
// Work decomposition (one workgroup = NW waves = 32*NW queries of one (batch, head); NW = 8 or
// 4, chosen per launch by how well the grid fills the CUs):
//   * each wave owns 32 queries and keeps them in registers as the B operand of
//     v_mfma_f32_32x32x16_bf16, computing S^T = K Q^T so that one lane holds one query's
//     scores; the softmax row statistics then need one lane-pair swap (v_permlane32_swap);
//   * the row max is not recomputed per tile: probabilities are formed as
//     exp2(s * scale * log2(e) - m) with the running max m (one fma, one v_exp_f32, one add
//     and half a bf16 pack per score), and a tile whose probabilities could exceed 2^8
//     (detected from the lane's partial sum) takes a rare path that raises the max to the
//     tile's true max, recomputes the tile and rescales O;
//   * 64-key K and V^T tiles are staged in LDS and shared by the waves, in MFMA operand order
//     (see kBlockBytes), by buffer loads straight into LDS: one descriptor per tile, the
//     lane's byte offset in a VGPR that never changes, the block offset in an SGPR.  K is
//     staged two tiles ahead and V one tile ahead of their use (three and one on the
//     four-buffer ring of 8-wave groups over 2-byte pools, with a barrier every second tile);
//   * the K rows of each 32-key block are loaded in the permuted order key_perm(), which makes
//     the fp32 S^T accumulator of a lane hold, per 8 registers, 8 consecutive keys — exactly
//     the bf16x8 B operand (P^T) of the PV product; V is stored transposed in the pool so
//     its A operand (V^T rows) is one 16 B LDS read;
//   * iteration tau runs three independent streams — QK(tau+1), softmax(tau), PV(tau-1) —
//     interleaved by hand (one MFMA, then a slice of the softmax) so the matrix core and the
//     VALU work at the same time; the softmax is front-loaded so its row sum is ready when the
//     last MFMA issues; the loop is unrolled twice so score and probability registers
//     alternate between two sets instead of being copied;
//   * tiles either follow frames (each frame padded to whole 64-token tiles) or, for whole
//     bf16 / f16 frames of 8k tokens without RoPE, run across frame boundaries (PK: a tile's
//     keys end one frame's slot and start the next one's); padding keys and keys beyond a
//     query's chunk-causal limit get -inf, decided per tile: full tiles skip the mask, tiles
//     past every query's limit are not visited.

#include <math.h>

#include <algorithm>
#include <type_traits>
#include <utility>

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
  // key tiles per q-tile: n_frames * ntiles_f, or ceil(n_keys / 64) when the tiles are packed
  // across frame boundaries (attn_kernel<..., PK = true>)
  int nt;
  int packed;  // 1: the bf16 / f16 kernels run their packed-tile instance
  // bytes of each pool when packed (< 4 GB): the range of the packed kernel's buffer descriptors,
  // so that no offset can reach past the pool
  uint32_t pool_bytes;
  float scale_log2;  // softmax_scale * log2(e)
  int mask_mode;
  int64_t q_pos0, chunk, n_keys;
  // RoPE on load (bf16 pools; kpool is then the height/width-roped K copy): rope_hw = cos, sin
  // per (h, pair) then per (w, pair) of the spatial pairs; rope_t = cos, sin of
  // (p_query_frame - p_key_frame) * w_j per (query frame, key frame, temporal pair)
  const float* rope_hw;
  const float* rope_t;
  int gh, gw, n_qframes;
  // PRoPE (camera transforms, applied after RoPE) on the same path; every matrix is a row-major
  // 4x4 acting on one group of 4 consecutive head channels:
  //   pq_t [B][n_frames][n_qframes][11][16]: W = R_k^T (P_q P_k^-1)^T R_q per temporal group
  //        (applied to the raw query; R = that group's temporal RoPE rotation at p_key / p_query)
  //   pq_s [B][n_qframes][16]: P_q^T, applied to the query's spatial groups after their RoPE
  //   pq_o [B][n_qframes][16]: P_q, applied to every group of the output
  const float* pq_t;
  const float* pq_s;
  const float* pq_o;
  // RMSNorm of Q at load (the reference's norm_q): row r of stream b is scaled by
  // q_rms[b * q_rms_sb + r] and channel h*D + c by q_w[h*D + c] (fp32); nullptr = Q as given
  const float* q_rms;
  int64_t q_rms_sb;
  const float* q_w;
  int32_t slots[SKV_MAX_FRAMES];
  // valid keys of each listed frame (T unless the caller gives ragged frames, e.g. a prefix span
  // stored in partly filled slots); keys t >= flen[j] of frame j are masked.  32-bit so a
  // wave-uniform index reads it with a scalar load.
  int32_t flen[SKV_MAX_FRAMES];
  // Balanced key split (no mask, 8-wave groups): the n_wg workgroups share the
  // units = B*H*n_qtiles*nt (q-tile, key tile) pairs equally; workgroup i
  // takes units [i*units/n_wg, (i+1)*units/n_wg) in q-tile order.  A q-tile that one workgroup
  // covers whole is written directly; a part of a split q-tile goes to record 2i (the
  // workgroup's first segment) or 2i+1 (its last) of part_o / part_ml, and attn_combine_kernel
  // merges the records of each split q-tile.
  int split;
  int64_t units;
  // q-tile (in (b, h)-major order) that unit 0 / workgroup 0 of this grid starts at: 0, except
  // for the tail launch of a grid whose last round is split (the full rounds run unsplit first)
  int qt_base;
  float* part_o;   // [2*n_wg][256][128] unnormalised O
  float* part_ml;  // [2*n_wg][256][2] (running max in log2 units, row sum)
  // Segments (the SEG instances; n_seg = 0 otherwise): the queries are n_seg consecutive row
  // ranges of seg_rows[s] rows, each attending its own seg_nf[s] consecutive entries of the
  // frame list; a segment's q-tiles start at its first row, n_qtiles counts them all.
  int n_seg;
  int32_t seg_rows[SKV_MAX_SEGMENTS];
  int32_t seg_nf[SKV_MAX_SEGMENTS];
};

// Wan's split of a head's 64 complex channel pairs (2i, 2i+1): 22 temporal, 21 height, 21 width
// (causal_model.py:1855-1866).
constexpr int kRopeT = 22, kRopeHW = 21;
constexpr int kGroupsT = kRopeT / 2;  // PRoPE groups (4 channels) holding temporal pairs only
// PRoPE: the W matrices of one key frame for the workgroup's query frames (at most 5 when
// frame_tokens >= 64) are staged in LDS behind the K/V tiles, double-buffered by frame parity.
constexpr int kWPair = kGroupsT * 16 * 4;  // bytes of W per (query frame, key frame)
constexpr int kWMaxQF = 5;
constexpr int kWBuf = 4096;                // >= kWMaxQF * kWPair, whole 1 KB wave chunks
static_assert(kWMaxQF * kWPair <= kWBuf, "W buffer too small");

// y[4g .. 4g+4) <- m (row-major 4x4) x y[4g .. 4g+4)
__device__ inline void xform4(Vec8<float>& y, int g, const float* m) {
  const float x0 = y.get(4 * g), x1 = y.get(4 * g + 1), x2 = y.get(4 * g + 2), x3 = y.get(4 * g + 3);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    y.set(4 * g + i, fmaf(m[4 * i], x0, fmaf(m[4 * i + 1], x1, fmaf(m[4 * i + 2], x2, m[4 * i + 3] * x3))));
}

// Workgroups have NW = 4 or 8 waves (128 or 256 queries); the launcher picks the shape that
// fills the 256 CUs best (8-wave groups halve the K/V bytes staged per query).

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

// PV step st (0..15) of a tile: O block db += V^T(db, kb, s2) P^T(kb, s2), the four O blocks in
// turn so consecutive PV MFMAs never accumulate into the same block (each block still sums its
// four products in the order (kb, s2) = (0,0), (0,1), (1,0), (1,1))
__device__ inline void pv_order(int st, int& db, int& kbb, int& s2) {
  db = st & 3, kbb = (st >> 3) & 1, s2 = (st >> 2) & 1;
}

// Combine a lane's value with lane l^32's (the other key half of the same query) using the
// gfx950 VALU lane swap; for a symmetric op both outputs of the swap pair give the result.
__device__ inline float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The frame list a walk reads: entries [fb, fb + nf) of the launch's list.  A plain launch walks
// the whole list (no state: fb is 0 and nf the launch's frame count); a segmented launch walks its
// segment's sub-list, set when the work-group has found its segment.
template <bool SEG>
struct FrameRange {
  __device__ int fb() const { return 0; }
  __device__ int nf(const AttnArgs& a) const { return a.n_frames; }
  __device__ void range(int, int) {}
};

template <>
struct FrameRange<true> {
  int b = 0, n = 0;
  __device__ int fb() const { return b; }
  __device__ int nf(const AttnArgs&) const { return n; }
  __device__ void range(int first, int count) { b = first; n = count; }
};

// Walks key tiles in frame-list order.  The frame's pool offset and valid length are read when
// the walk enters the frame, so advancing by one tile costs a few scalar adds: no division by
// the tiles per frame and no table load on the tiles in between.  Every member is wave-uniform.
template <bool SEG = false>
struct TileWalk : FrameRange<SEG> {
  int j = 0, t = 0;   // frame index in the walked list, tile inside the frame
  int32_t slot = 0;   // the frame's slot
  int64_t base = 0;   // element offset of frame j's (b, h) block: slot * slot_stride + kbh
  int flen = 0;       // valid keys of frame j
  __device__ void open(const AttnArgs& a, int64_t kbh) {
    if (j < this->nf(a)) {
      slot = a.slots[this->fb() + j];
      base = (int64_t)slot * a.slot_stride + kbh;
      flen = a.flen[this->fb() + j];
    }
  }
  __device__ void start(const AttnArgs& a, int64_t kbh, int tg) {
    j = tg / a.ntiles_f;
    t = tg - j * a.ntiles_f;
    open(a, kbh);
  }
  __device__ void next(const AttnArgs& a, int64_t kbh) {
    if (++t == a.ntiles_f) {
      t = 0;
      ++j;
      open(a, kbh);
    }
  }
};

// Walks 64-key tiles packed across frame boundaries: tile g holds keys [64 g, 64 g + 64) of the
// window (frames of T tokens end to end, no padding keys), so it may straddle frames j and j + 1:
// its first T - t0 keys are tokens t0.. of frame j, the rest tokens 0.. of frame j + 1.  Offsets
// are bytes from the pool's start (the host packs only pools under 4 GB), read when the walk
// enters frame j; advancing by one tile costs a few scalar ops.  Past the last frame, off_n
// repeats off (the keys there are masked and their rows are only read, in bounds, so that the
// staged values stay finite).  Every member is wave-uniform.
template <bool SEG = false>
struct PackedWalk : FrameRange<SEG> {
  int j = 0, t0 = 0;
  uint32_t off = 0, off_n = 0;  // byte offsets of frames j and j + 1's (b, h) blocks
  __device__ void open(const AttnArgs& a, int64_t kbh) {
    const int nf = this->nf(a), fb = this->fb();
    if (j < nf) {
      off = (uint32_t)(((int64_t)a.slots[fb + j] * a.slot_stride + kbh) * 2);
      off_n = j + 1 < nf ? (uint32_t)(((int64_t)a.slots[fb + j + 1] * a.slot_stride + kbh) * 2) : off;
    }
  }
  __device__ void start(const AttnArgs& a, int64_t kbh, int g) {
    const int key0 = g * kTile;
    j = key0 / a.T;
    t0 = key0 - j * a.T;
    open(a, kbh);
  }
  __device__ void next(const AttnArgs& a, int64_t kbh) {
    t0 += kTile;
    if (t0 >= a.T) {
      t0 -= a.T;
      ++j;
      open(a, kbh);
    }
  }
};

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

template <>
__device__ inline void store4<f16>(f16* p, float x0, float x1, float x2, float x3) {
  typedef f16 f16x4 __attribute__((ext_vector_type(4)));
  f16x4 v;
  v[0] = (f16)x0; v[1] = (f16)x1; v[2] = (f16)x2; v[3] = (f16)x3;
  *reinterpret_cast<f16x4*>(p) = v;
}

// Stage one 64-key tile of K (or V^T) into a 16 KB LDS buffer: wave w writes operand blocks
// [w*kBpw, (w+1)*kBpw) of the 16.  K block b = (kb = b/8, k-step s = b%8); V^T block
// b = (db = b/4, kb*2+s2 = b%4).  bf16 pools use direct 16 B global->LDS loads (no registers);
// fp32 pools (the C1 path, not performance critical) go through registers and are rounded.
// fp8-e4m3 pool element (one code byte) for attn_kernel's RoPE / PRoPE instances, which decode
// each staged tile to bf16 with its frame's scale and multiply in bf16.
struct fp8e4 {
  uint8_t v;
};

// 8 e4m3 codes -> 8 bf16 of code x scale (fp32 product, one rounding to bf16)
__device__ inline bf16x8 decode_e4m3x8(const u32x2& w, float sc) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
    r[4 * i] = (bf16)(lo[0] * sc);
    r[4 * i + 1] = (bf16)(lo[1] * sc);
    r[4 * i + 2] = (bf16)(hi[0] * sc);
    r[4 * i + 3] = (bf16)(hi[1] * sc);
  }
  return r;
}

template <int NW, typename KT>
struct TileLoader {
  static constexpr int kBpw = 16 / NW;
  int64_t koff, voff;   // element offsets of this lane's first block (register path)
  uint32_t klane, vlane;  // byte offsets of this lane inside a block (buffer path)
  int wu, Tp;
  int lane16;
  int kk_k;  // key (inside the tile) of this lane's K rows: the same in all of the wave's blocks
  int hh8;   // first of the lane's 8 tokens inside a V^T block's 16-key step
  // packed tiles: the lane's byte offset inside the tile for each of the wave's K / V^T blocks
  // (lane part + block part), so that a load adds only the tile's offset
  uint32_t kpk[kBpw], vpk[kBpw];
  __device__ void init(int w, int lane, int Tp_) {
    lane16 = lane * 16;
    Tp = Tp_;
    wu = __builtin_amdgcn_readfirstlane(w);
    const int n = lane & 31, hh = lane >> 5;
    const int b0 = w * kBpw;
    koff = (int64_t)((b0 >> 3) * 32 + key_perm(n)) * kHeadDim + (b0 & 7) * 16 + hh * 8;
    voff = (int64_t)((b0 >> 2) * 32 + n) * Tp + (b0 & 3) * 16 + hh * 8;
    klane = (uint32_t)(key_perm(n) * kHeadDim + hh * 8) * 2u;
    vlane = (uint32_t)(n * Tp + hh * 8) * 2u;
    kk_k = (b0 >> 3) * 32 + key_perm(n);
    hh8 = hh * 8;
#pragma unroll
    for (int j = 0; j < kBpw; ++j) {  // after klane / vlane, which they extend
      const int b = b0 + j;
      kpk[j] = klane + (uint32_t)((b >> 3) * 32 * kHeadDim + (b & 7) * 16) * 2u;
      vpk[j] = vlane + (uint32_t)((b >> 2) * 32 * Tp + (b & 3) * 16) * 2u;
    }
  }
  // bf16 pools: one buffer descriptor per tile (base = the tile's first element), the lane's
  // byte offset in a VGPR that never changes, the block's offset in an SGPR.
  __device__ void issue_k(const KT* kt, char* dst, int w) const {
    if constexpr (sizeof(KT) == 2) {
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)kt, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
      for (int j = 0; j < kBpw; ++j) {
        const int b = wu * kBpw + j;
        const uint32_t so = (uint32_t)((b >> 3) * 32 * kHeadDim + (b & 7) * 16) * 2u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + b * kBlockBytes), 16, klane, so, 0, 0);
      }
    } else if constexpr (sizeof(KT) == 4) {
      dst += w * kBpw * kBlockBytes;
#pragma unroll
      for (int j = 0; j < kBpw; ++j) stage(kt + koff + j * 16, dst + j * kBlockBytes);
    }
  }
  __device__ void issue_v(const KT* vt, char* dst, int w) const {
    if constexpr (sizeof(KT) == 2) {
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)vt, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
      for (int j = 0; j < kBpw; ++j) {
        const int b = wu * kBpw + j;
        const uint32_t so = (uint32_t)((b >> 2) * 32 * Tp + (b & 3) * 16) * 2u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + b * kBlockBytes), 16, vlane, so, 0, 0);
      }
    } else if constexpr (sizeof(KT) == 4) {
      dst += w * kBpw * kBlockBytes;
#pragma unroll
      for (int j = 0; j < kBpw; ++j) stage(vt + voff + j * 16, dst + j * kBlockBytes);
    }
  }
  __device__ void stage(const KT* src, char* block) const {
    *reinterpret_cast<bf16x8*>(block + lane16) = Vec8<KT>::load(src).to_bf16();
  }
  // fp8 pools: the lane's 8 codes of each of the wave's K / V^T blocks, fetched into registers
  // at a step's start and decoded into the LDS blocks at its end, so the loads' latency is
  // covered by the step's products
  // (buffer loads: one descriptor per tile in SGPRs, the lane's byte offset in a VGPR that never
  // changes, so no 64-bit address per lane and block)
  u32x2 kraw[kBpw], vraw[kBpw];
  __device__ void fetch_k(const KT* kt) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)kt, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int j = 0; j < kBpw; ++j)
      kraw[j] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)koff, j * 16, 0));
  }
  __device__ void fetch_v(const KT* vt) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)vt, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int j = 0; j < kBpw; ++j)
      vraw[j] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, j * 16, 0));
  }
  __device__ void commit_k(char* dst, int w, float sc) const {
    dst += w * kBpw * kBlockBytes + lane16;
#pragma unroll
    for (int j = 0; j < kBpw; ++j)
      *reinterpret_cast<bf16x8*>(dst + j * kBlockBytes) = decode_e4m3x8(kraw[j], sc);
  }
  __device__ void commit_v(char* dst, int w, float sc) const {
    dst += w * kBpw * kBlockBytes + lane16;
#pragma unroll
    for (int j = 0; j < kBpw; ++j)
      *reinterpret_cast<bf16x8*>(dst + j * kBlockBytes) = decode_e4m3x8(vraw[j], sc);
  }
  // Packed tiles (2-byte pools), through one descriptor over the whole pool: the tile's keys
  // kk < bnd come from frame j (byte offset oa of the tile's first key, token t0), the others
  // from frame j + 1 (on: its first token's offset less bnd tokens, so that the same lane
  // offsets apply).  A tile inside one frame (bnd >= 64) adds oa to each block's scalar offset;
  // a straddling tile puts the lane's whole offset in its VGPR (formed modulo 2^32: a lane of
  // frame j + 1 lies at least bnd tokens past `on`, so the sum is its true offset), the loads
  // stay wave-uniform.  V^T's 8-token groups never straddle (T, t0 multiples of 8).
  __device__ void issue_k_packed(const KT* pool, uint32_t nbytes, uint32_t oa, uint32_t on, int bnd,
                                 char* dst) const {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass would drop the calling kernels' launch stubs
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)pool, (short)0, (int)nbytes, 0x00020000);
    // an opaque copy of the wave index: the blocks' LDS addresses are formed here, by scalar
    // adds, instead of hoisted out of the main loop as 4 long-lived SGPRs per operand
    int wq = wu;
    asm volatile("" : "+s"(wq));
    if (bnd >= kTile) {
#pragma unroll
      for (int j = 0; j < kBpw; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + (wq * kBpw + j) * kBlockBytes), 16,
                                                 kpk[j], oa, 0, 0);
    } else {
      const uint32_t o = kk_k < bnd ? oa : on;
#pragma unroll
      for (int j = 0; j < kBpw; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + (wq * kBpw + j) * kBlockBytes), 16,
                                                 kpk[j] + o, 0, 0, 0);
    }
#endif
  }
  __device__ void issue_v_packed(const KT* pool, uint32_t nbytes, uint32_t oa, uint32_t on, int bnd,
                                 char* dst) const {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass would drop the calling kernels' launch stubs
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)pool, (short)0, (int)nbytes, 0x00020000);
    int wq = wu;
    asm volatile("" : "+s"(wq));
    if (bnd >= kTile) {
#pragma unroll
      for (int j = 0; j < kBpw; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + (wq * kBpw + j) * kBlockBytes), 16,
                                                 vpk[j], oa, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < kBpw; ++j) {
        const int b = wu * kBpw + j;  // wu: the lane-offset choice, a constant per block
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + (wq * kBpw + j) * kBlockBytes), 16,
                                                 vpk[j] + ((b & 3) * 16 + hh8 < bnd ? oa : on), 0, 0, 0);
      }
    }
#endif
  }
};

// MFMA operand element of a pool type: f16 pools multiply in f16, every other pool (bf16, and
// fp32 rounded to bf16 on staging) in bf16.
template <typename KT>
struct OpOf {
  using E = bf16;
  using x8 = bf16x8;
  template <typename V>
  __device__ static x8 from(const V& v) { return v.to_bf16(); }
};
template <>
struct OpOf<f16> {
  using E = f16;
  using x8 = f16x8;
  template <typename V>
  __device__ static x8 from(const V& v) { return v.to_f16(); }
};
__device__ inline f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ inline f32x16 mfma32(const f16x8& a, const f16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// S^T (64 keys x 32 queries of this wave) = K Q^T from a K tile in LDS.
template <typename X8>
__device__ inline void qk_tile(const char* kl, const X8 (&qf)[8], f32x16 (&s)[2]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s[kb][i] = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const X8 ak = *reinterpret_cast<const X8*>(kl + (kb * 8 + k) * kBlockBytes);
      s[kb] = mfma32(ak, qf[k], s[kb]);
    }
  }
}

// Padding keys (token >= T inside the frame) and keys past the lane's chunk-causal limit.
// x = -inf unless C < t: one compare into vcc and one select per register, written as one asm
// statement so the compares are not hoisted ahead of the selects (32 live SGPR pairs spill)
template <int C>
__device__ inline float mask_below(float x, int t, float ninf) {
  asm("v_cmp_lt_i32 vcc, %2, %1\n\tv_cndmask_b32 %0, %3, %0, vcc"
      : "+v"(x) : "v"(t), "n"(C), "v"(ninf) : "vcc");
  return x;
}
// register I of a tile's two accumulators (s[I >> 4][I & 15]) holds key offset KeyOf(I)
template <template <int> class KeyOf, int... I>
__device__ inline void mask_regs(f32x16 (&s)[2], int t, std::integer_sequence<int, I...>) {
  const float ninf = -INFINITY;
  ((s[I >> 4][I & 15] = mask_below<KeyOf<I>::value>(s[I >> 4][I & 15], t, ninf)), ...);
}
template <int I>
struct KeyBf16 : std::integral_constant<int, (I >> 4) * 32 + ((I & 15) >> 3) * 16 + (I & 7)> {};
template <int I>
struct KeyFp8 : std::integral_constant<int, I> {};

__device__ inline void mask_tile(f32x16 (&s)[2], int hh, int tok0, int T, int key0, int lim) {
  // key kk of the tile is masked when tok0 + kk >= T or key0 + kk >= lim, i.e. when
  // kk >= min(T - tok0, lim - key0); kk = 8 hh + c with c fixed per register, so each register
  // takes one compare against a constant
  const int t = min(T - tok0, lim - key0) - 8 * hh;
  mask_regs<KeyBf16>(s, t, std::make_integer_sequence<int, 32>{});
}

// K and V^T tile buffers of attn_kernel's ring: 4 (a barrier every second step) for 8-wave groups
// over 2-byte pools, 2 otherwise: 4-wave groups run two workgroups per CU, whose 2 x 128 KB would
// not fit the 160 KB of LDS; fp32 pools and the frame-aligned split spill registers with the
// longer ring.
constexpr int attn_ring(int nw, int rm, int kt_bytes, bool split, bool pk) {
  return nw == 8 && kt_bytes == 2 && (pk || !split) ? 4 : 2;
}
// PRoPE matrix buffers: one per key frame in flight (frame j in buffer j mod n); with the longer
// ring a frame's matrices are staged three steps before use, so frames of a single tile need four
constexpr int attn_wbufs(int ring) { return ring == 4 ? 4 : 2; }
constexpr size_t attn_lds_bytes(int nw, int rm, int kt_bytes, bool split, bool pk) {
  return (size_t)attn_ring(nw, rm, kt_bytes, split, pk) * kTileBytes +
         (rm == 2 ? (size_t)attn_wbufs(attn_ring(nw, rm, kt_bytes, split, pk)) * kWBuf : 0);
}

// PK: key tiles packed across frame boundaries (PackedWalk; whole frames of T = 8k tokens, 2-byte
// pools, no RoPE): a window of n frames takes ceil(n T / 64) tiles instead of n ceil(T / 64).
// SEG: the grid's q-tiles belong to consecutive query segments, each over its own slice of the
// frame list (AttnArgs::n_seg); no RoPE, no mask, no split.
template <int NW, typename QT, typename KT, int RM, bool SPLIT = false, bool PK = false,
          bool SEG = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_kernel(AttnArgs a) {
  static_assert(!PK || (RM == 0 && sizeof(KT) == 2), "packed tiles: 2-byte pools, no RoPE");
  static_assert(!SEG || (RM == 0 && !SPLIT), "segments: no RoPE, no split");
  constexpr int kBQ = NW * 32;
  // LDS map: kRing K buffers, then kRing V^T buffers (tile x in buffer x mod kRing), then (PRoPE)
  // kWN matrix buffers.  A step reads K(tau+1) and V(tau-1) and loads K(tau+kL+1) and V(tau+kL-1);
  // the workgroup meets at a barrier after every kL-th step.  kL = 1 (two buffers each) for
  // 4-wave groups (two workgroups share a CU's LDS), fp32 pools and the frame-aligned split;
  // the others take kL = 2.
  constexpr int kRing = attn_ring(NW, RM, (int)sizeof(KT), SPLIT, PK);
  constexpr int kL = kRing / 2;
  constexpr int kWN = attn_wbufs(kRing);
  using ET = typename OpOf<KT>::E;     // MFMA operand element
  using etx8 = typename OpOf<KT>::x8;
  // LDS: K tiles in [0, 32 KB) (two buffers), V^T tiles in [32 KB, 64 KB) (two buffers).
  extern __shared__ __attribute__((aligned(16))) char lds[];
  constexpr int kHalf = 16 * kBlockBytes;

  // XCD-aware order: workgroup ids are dealt round-robin over the 8 XCDs; XCD x gets the
  // contiguous logical range starting at x*per + min(x, rem), so q-tiles of one head run on
  // one XCD and stream the same K/V through its L2.
  int logical;
  {
    const int bid = blockIdx.x, xcd = bid & 7, idx = bid >> 3;
    const int per = a.n_wg >> 3, rem = a.n_wg & 7;
    logical = xcd * per + min(xcd, rem) + idx;
  }
  // Segments: key tiles [tb, te) of q-tile qg; one whole q-tile unless split.  A split share
  // [u0, u1) covers q-tiles q_first .. q_first + nseg - 1 (segment j = q-tile q_first + j); the
  // whole ones run first, then the last segment (key tiles from 0, in step with the other
  // workgroups, which all start at key tile 0), then the first (the tail of a q-tile, a fixed
  // number of tiles ahead of them): K/V tiles stay shared through L2 as in the unsplit grid.
  const int nt = a.nt;
  int q_first = logical, nseg = 1;
  int64_t u0 = 0, u1 = 0;
  if constexpr (SPLIT) {
    u0 = (int64_t)logical * a.units / a.n_wg;
    u1 = (int64_t)(logical + 1) * a.units / a.n_wg;
    q_first = (int)(u0 / nt);
    nseg = u1 > u0 ? (int)((u1 - 1) / nt) - q_first + 1 : 0;
  }
  for (int k = 0; k < nseg; ++k) {
  const int seg = nseg == 1 ? 0 : k < nseg - 2 ? k + 1 : k == nseg - 2 ? nseg - 1 : 0;
  const int qg = q_first + seg;
  int tb = 0, te = nt;
  if constexpr (SPLIT) {
    if (seg == 0) tb = (int)(u0 - (int64_t)q_first * nt);
    if (seg == nseg - 1) te = (int)(u1 - (int64_t)qg * nt);
  }
  if (k > 0) __syncthreads();  // the previous segment's last LDS reads are done
  const int qt = (qg + a.qt_base) % a.n_qtiles;
  const int bh = (qg + a.qt_base) / a.n_qtiles;
  const int h = bh % a.H, b = bh / a.H;
  // the q-tile's query rows [qr0 + qtl * kBQ, ...) < qend and its frame list [fb, fb + nfr)
  int qr0 = 0, qend = a.Lq, qtl = qt, fb = 0, nfr = a.n_frames;
  if constexpr (SEG) {
    // q-tiles are dealt last segment first: later segments attend longer lists in the callers'
    // layouts (teacher forcing, memory KV), so the longest work-groups start first
    qtl = a.n_qtiles - 1 - qt;
    qend = 0;
    for (int sg = 0; sg < a.n_seg; ++sg) {  // wave-uniform scan of the segment table
      const int rows = a.seg_rows[sg], nq = (rows + kBQ - 1) / kBQ;
      qr0 = qend;
      qend += rows;
      nfr = a.seg_nf[sg];
      if (qtl < nq) break;
      qtl -= nq;
      fb += nfr;
    }
  }

  // SPLIT: an opaque copy per segment, so lane-derived values are recomputed here instead of
  // hoisted out of the segment loop, where they would stay live through the tile loop
  int tid = threadIdx.x;
  if constexpr (SPLIT) asm volatile("" : "+v"(tid));
  const int lane = tid & 63, w = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int q0 = qr0 + qtl * kBQ;
  const int qrow = q0 + w * 32 + n;
  const bool qlive = qrow < qend;

  // Q^T operand: lane (n, hh) holds q[qrow][k*16 + hh*8 .. +7] for k = 0..7.
  etx8 qf[8];
  // RM = 0: Q as given.  RM = 1 (RoPE): the query's height/width pairs are rotated once here;
  // its temporal pairs (0..21, in qf[0..2]) are kept unrotated in qt0 and turned by
  // (p_query - p_key) per key frame below.  RM = 2 (RoPE + PRoPE): as RM = 1, the spatial
  // groups then take P_q^T, and the temporal groups take the per-key-frame matrix W below.
  [[maybe_unused]] etx8 qt0[3];
  [[maybe_unused]] int qfi = 0;  // query frame of this lane's row
  {
    const QT* qp = static_cast<const QT*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                   (int64_t)(qlive ? qrow : 0) * a.q_st + hh * 8;
    // RMSNorm factor of this row (0 for dead rows) and its channel weights
    const float qn = a.q_rms && qlive ? a.q_rms[(int64_t)b * a.q_rms_sb + qrow] : 0.f;
    const float* qw = a.q_w + h * kHeadDim + hh * 8;
    if constexpr (RM > 0) {
      const int qr = qlive ? qrow : a.Lq - 1;
      qfi = qr / a.T;
      const int tt = qr - qfi * a.T, hq = tt / a.gw, wq = tt - hq * a.gw;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const Vec8<QT> x = qlive ? Vec8<QT>::load(qp + k * 16) : Vec8<QT>::zero();
        Vec8<float> y;
        if (a.q_rms) {
#pragma unroll
          for (int e = 0; e < 8; ++e) y.set(e, (float)x.get(e) * qn * qw[k * 16 + e]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) y.set(e, (float)(bf16)x.get(e));
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int pr = k * 8 + hh * 4 + m;
          if (pr < kRopeT) continue;
          const int idx = pr < kRopeT + kRopeHW ? hq * kRopeHW + (pr - kRopeT)
                                                : (a.gh + wq) * kRopeHW + (pr - kRopeT - kRopeHW);
          const float c = a.rope_hw[2 * idx], sn = a.rope_hw[2 * idx + 1];
          const float u = y.get(2 * m), v = y.get(2 * m + 1);
          y.set(2 * m, u * c - v * sn);
          y.set(2 * m + 1, u * sn + v * c);
        }
        if constexpr (RM == 2) {
          const float* ps = a.pq_s + ((int64_t)b * a.n_qframes + qfi) * 16;
#pragma unroll
          for (int gg = 0; gg < 2; ++gg)
            if (4 * k + 2 * hh + gg >= kGroupsT) xform4(y, gg, ps);
        }
        qf[k] = OpOf<KT>::from(y);
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) qt0[k] = qf[k];
    } else if (a.q_rms) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const Vec8<QT> x = qlive ? Vec8<QT>::load(qp + k * 16) : Vec8<QT>::zero();
        Vec8<float> y;
#pragma unroll
        for (int e = 0; e < 8; ++e) y.set(e, (float)x.get(e) * qn * qw[k * 16 + e]);
        qf[k] = OpOf<KT>::from(y);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        qf[k] = OpOf<KT>::from(qlive ? Vec8<QT>::load(qp + k * 16) : Vec8<QT>::zero());
    }
  }
  // PRoPE: W of key frame j for query frames [qf_lo, qf_lo + count) -> LDS buffer j & 1 (waves
  // 0..3 move 1 KB each with direct global->LDS loads; completion is awaited with the tiles')
  [[maybe_unused]] const int qf_lo = q0 / a.T;
  [[maybe_unused]] auto issue_w = [&](int j) {
    if constexpr (RM == 2) {
      const int count = (min(q0 + kBQ, a.Lq) - 1) / a.T - qf_lo + 1;
      const int off = w * 1024 + lane * 16;
      if (w < kWBuf / 1024 && off < count * kWPair) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.pq_t, (short)0, 0x7fffffff, 0x00020000);
        const uint32_t so = (uint32_t)((((int64_t)b * a.n_frames + j) * a.n_qframes + qf_lo) * kWPair);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (lds_void_t*)(lds + kRing * kTileBytes + (j % kWN) * kWBuf + w * 1024), 16, off, so, 0, 0);
      }
    }
  };
  // qf[0..2] <- qt0 with the temporal pairs turned by the angle of (query frame, key frame j)
  // (RM = 1), or with each temporal group multiplied by that pair's W (RM = 2)
  [[maybe_unused]] auto rot_q = [&](int j) {
    if constexpr (RM == 2) {
      // W of (this lane's query frame, key frame j), staged in LDS by issue_w; one group's
      // rows are live at a time (this runs inside the main loop, where registers are scarce)
      const float* wt = reinterpret_cast<const float*>(lds + kRing * kTileBytes + (j % kWN) * kWBuf) +
                        (qfi - qf_lo) * (kGroupsT * 16);
#pragma unroll
      for (int k = 0; k < 3; ++k) {
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
          const int g = 4 * k + 2 * hh + gg;
          if (g >= kGroupsT) continue;
          // an opaque copy keeps the loop-invariant bf16 -> fp32 conversion here instead of
          // hoisted out of the main loop (24 live floats there would spill)
          bf16x8 t = qt0[k];
          asm volatile("" : "+v"(t));
          float x[4], r[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = (float)t[4 * gg + e];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float4 m = *reinterpret_cast<const float4*>(wt + g * 16 + 4 * i);
            r[i] = fmaf(m.x, x[0], fmaf(m.y, x[1], fmaf(m.z, x[2], m.w * x[3])));
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) qf[k][4 * gg + e] = (bf16)r[e];
          asm volatile("" ::: "memory");
        }
      }
      return;
    }
    const float* tb = a.rope_t + ((int64_t)qfi * a.n_frames + j) * (2 * kRopeT);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      Vec8<float> y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y.set(e, (float)qt0[k][e]);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int pr = k * 8 + hh * 4 + m;
        if (pr >= kRopeT) continue;
        const float c = tb[2 * pr], sn = tb[2 * pr + 1];
        const float u = y.get(2 * m), v = y.get(2 * m + 1);
        y.set(2 * m, u * c - v * sn);
        y.set(2 * m + 1, u * sn + v * c);
      }
      qf[k] = OpOf<KT>::from(y);
    }
  };

  // Visibility limits (keys indexed 0..n_keys-1 in frame-list order; n_keys < 2^31).
  const int n_keys = SEG ? nfr * a.T : (int)a.n_keys;
  int lim_lane = n_keys, lim_lo = n_keys, lim_hi = n_keys;
  if (a.mask_mode == SKV_MASK_CHUNK_CAUSAL) {
    const int qlast = min(q0 + kBQ, a.Lq) - 1;
    lim_lane = (int)chunk_limit(a.q_pos0 + min(qrow, a.Lq - 1), a.chunk, n_keys);
    lim_lo = (int)chunk_limit(a.q_pos0 + q0, a.chunk, n_keys);
    lim_hi = (int)chunk_limit(a.q_pos0 + qlast, a.chunk, n_keys);
  }
  int ntau;
  {
    const int jf = lim_hi / a.T;
    ntau = jf >= nfr ? nfr * a.ntiles_f : jf * a.ntiles_f + (lim_hi - jf * a.T + kTile - 1) / kTile;
    if constexpr (PK) ntau = (lim_hi + kTile - 1) / kTile;  // lim_hi <= n_keys
    if constexpr (SPLIT) ntau = te - tb;  // no mask: the segment's tiles
  }

  const KT* kpool = static_cast<const KT*>(a.kpool);
  const KT* vpool = static_cast<const KT*>(a.vpool);
  const int64_t kbh = (int64_t)(b * a.H + h) * a.Tp * kHeadDim;  // (b,h) offset inside a slot
  TileLoader<NW, KT> loader;
  loader.init(w, lane, a.Tp);
  auto tile_base = [&](int tau) -> int64_t {
    const int tg = tb + tau, j = tg / a.ntiles_f, t = tg - j * a.ntiles_f;
    return (int64_t)a.slots[fb + j] * a.slot_stride + kbh + (int64_t)t * kTile * kHeadDim;
  };
  [[maybe_unused]] auto tile_vbase = [&](int tau) -> int64_t {  // the same tile of V^T
    const int tg = tb + tau, j = tg / a.ntiles_f, t = tg - j * a.ntiles_f;
    return (int64_t)a.slots[fb + j] * a.slot_stride + kbh + (int64_t)t * kTile;
  };
  // fp8 pools: scales are [n_slots][B][H]; (b, h) of this workgroup is bh
  constexpr bool kFp8Pool = sizeof(KT) == 1;
  const int64_t n_bh = (int64_t)a.B * a.H;
  [[maybe_unused]] auto tile_scale = [&](const float* sc, int tau) -> float {
    const int j = (tb + tau) / a.ntiles_f;
    return sc[(int64_t)a.slots[fb + j] * n_bh + bh];
  };
  // mask decision for tile tau (uniform): returns true if any key of the tile may be hidden
  auto tile_needs_mask = [&](int tau, int& tok0, int& key0, int& tj) -> bool {
    const int tg = tb + tau, j = tg / a.ntiles_f, t = tg - j * a.ntiles_f;
    tok0 = t * kTile;
    key0 = j * a.T + tok0;
    tj = a.flen[fb + j];
    return (tok0 + kTile > tj) || (key0 + kTile > lim_lo);
  };
  // the same decision for the tile a walk stands on
  auto walk_needs_mask = [&](const TileWalk<SEG>& wk, int& tok0, int& key0) -> bool {
    tok0 = wk.t * kTile;
    key0 = wk.j * a.T + tok0;
    return (tok0 + kTile > wk.flen) || (key0 + kTile > lim_lo);
  };

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;
  // The fast path assumes a tile needs no new row max: p = exp2(s * c2 - m).  A lane whose
  // partial probability sum exceeds 2^kStale (or is not finite), or whose running max is
  // still -inf, sends the wave to the rare path, which raises the max to the tile's true max,
  // recomputes the tile's probabilities and rescales O and l.
  constexpr float kMaxPart = 256.0f;  // 2^kStale, kStale = 8
  float m_run = -INFINITY, l_run = 0.f;
  const float c2 = a.scale_log2;
  const int lane16 = lane * 16;
  auto kb_lds = [&](int i) { return lds + (i & (kRing - 1)) * kHalf; };
  auto vb_lds = [&](int i) { return lds + (kRing + (i & (kRing - 1))) * kHalf; };

  // Prologue: K(0..kL) and V(0..kL-2) resident; V(-1)'s buffer zeroed so PV(-1) of step 0 adds
  // nothing.
  // Score and probability registers ping-pong between two sets (A, B) across iterations, so no
  // loop-carried copy is needed.
  f32x16 sA[2], sB[2];
  etx8 pA[2][2], pB[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) pA[x][y] = OpOf<KT>::from(Vec8<float>::zero());
  f32x16 (&s_cur)[2] = sA;
  if (ntau > 0) {
    if constexpr (PK) {
      PackedWalk<SEG> p;
      p.range(fb, nfr);
      p.start(a, kbh, tb);
#pragma unroll
      for (int x = 0; x <= kL; ++x) {
        if (x < ntau)
          loader.issue_k_packed(kpool, a.pool_bytes, p.off + p.t0 * (kHeadDim * 2),
                                p.off_n - (a.T - p.t0) * (kHeadDim * 2), a.T - p.t0, kb_lds(x));
        p.next(a, kbh);
      }
      p.start(a, kbh, tb);
#pragma unroll
      for (int x = 0; x < kL - 1; ++x) {
        if (x < ntau)
          loader.issue_v_packed(vpool, a.pool_bytes, p.off + p.t0 * 2, p.off_n - (a.T - p.t0) * 2,
                                a.T - p.t0, vb_lds(x));
        p.next(a, kbh);
      }
    } else if constexpr (kFp8Pool) {
#pragma unroll
      for (int x = 0; x <= kL; ++x)
        if (x < ntau) {
          loader.fetch_k(kpool + tile_base(x));
          loader.commit_k(kb_lds(x), w, tile_scale(a.kscale, x));
        }
#pragma unroll
      for (int x = 0; x < kL - 1; ++x)
        if (x < ntau) {
          loader.fetch_v(vpool + tile_vbase(x));
          loader.commit_v(vb_lds(x), w, tile_scale(a.vscale, x));
        }
    } else {
#pragma unroll
      for (int x = 0; x <= kL; ++x)
        if (x < ntau) loader.issue_k(kpool + tile_base(x), kb_lds(x), w);
#pragma unroll
      for (int x = 0; x < kL - 1; ++x)
        if (x < ntau) loader.issue_v(vpool + tile_vbase(x), vb_lds(x), w);
    }
    if constexpr (RM == 2) {
      // matrices of the frames of tiles 0 .. kL (the steps stage those of later frames)
      issue_w(tb / a.ntiles_f);
#pragma unroll
      for (int x = 1; x <= kL; ++x)
        if (ntau > x && (tb + x) % a.ntiles_f == 0) issue_w((tb + x) / a.ntiles_f);
    }
#pragma unroll
    for (int r = 0; r < 16 / NW; ++r)
      *reinterpret_cast<bf16x8*>(vb_lds(-1) + (tid + NW * 64 * r) * 16) = Vec8<bf16>::zero().to_bf16();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if constexpr (RM > 0) rot_q(tb / a.ntiles_f);
    qk_tile(kb_lds(0) + lane16, qf, s_cur);
    if constexpr (PK) {
      const int key0 = tb * kTile;  // packed tiles hold no padding keys: only the limit masks
      if (key0 + kTile > lim_lo) mask_tile(s_cur, hh, 0, 1 << 30, key0, lim_lane);
    } else {
      int tok0, key0, tj;
      if (tile_needs_mask(0, tok0, key0, tj)) mask_tile(s_cur, hh, tok0, tj, key0, lim_lane);
    }
    __syncthreads();  // K(0) read by every wave before its buffer takes K(kRing)
  }

  // Iteration tau: QK(tau+1), softmax(tau) and PV(tau-1) are independent; their 32 MFMAs and
  // ~130 VALU ops are interleaved by hand (one MFMA, then a slice of the softmax) so the
  // matrix core and the VALU work at the same time.  Resident: K(tau+1), V(tau-1); in flight:
  // K(tau+2) into K(tau)'s buffer, V(tau) into V(tau-2)'s buffer.
  // cb = tau & 1, passed as a literal so buffer addresses fold into immediate offsets
  f32x16 zero16;
#pragma unroll
  for (int i = 0; i < 16; ++i) zero16[i] = 0.f;
  // Tiles addressed in step tau: K(tau+2) (kw), V(tau) (vw) and the mask / RoPE frame of
  // QK(tau+1) (mw); the walks advance one tile per step.
  TileWalk<SEG> kw, vw, mw;
  [[maybe_unused]] PackedWalk<SEG> kp, vp;
  kw.range(fb, nfr);
  vw.range(fb, nfr);
  mw.range(fb, nfr);
  kp.range(fb, nfr);
  vp.range(fb, nfr);
  if constexpr (PK) {
    kp.start(a, kbh, tb + kL + 1);
    vp.start(a, kbh, tb + kL - 1);
  } else {
    kw.start(a, kbh, tb + kL + 1);
    vw.start(a, kbh, tb + kL - 1);
    mw.start(a, kbh, tb + 1);
  }
  auto step = [&](int tau, const int cb, f32x16 (&s_cur)[2], f32x16 (&s_nxt)[2],
                  etx8 (&pprev)[2][2], etx8 (&pb)[2][2]) __attribute__((always_inline)) {
    // K(tau+1) (stale data on the last step) and V(tau-1) (zeros on the first step); with two
    // buffers the literal cb = tau & 1 names them, so their addresses fold into immediates
    const char* kl = (kRing == 2 ? kb_lds(cb ^ 1) : kb_lds(tau + 1)) + lane16;
    const char* vl = (kRing == 2 ? vb_lds(cb ^ 1) : vb_lds(tau - 1)) + lane16;
    // operand of MFMA slot i: even i -> QK step i/2 (k = i/4, kb = (i/2)&1), odd i -> PV step i/2
    auto operand = [&](int i) -> etx8 {
      const int st = i >> 1;
      if ((i & 1) == 0) {
        const int k = st >> 1, kbb = st & 1;
        return *reinterpret_cast<const etx8*>(kl + (kbb * 8 + k) * kBlockBytes);
      }
      int db, kbb, s2;
      pv_order(st, db, kbb, s2);
      return *reinterpret_cast<const etx8*>(vl + (db * 4 + kbb * 2 + s2) * kBlockBytes);
    };
    // the first three operands are requested before this step's loads are issued, so their LDS
    // latency overlaps the load set-up (PRoPE: after the query transform below, which needs the
    // registers)
    etx8 opq[4];
    if constexpr (RM != 2) {
#pragma unroll
      for (int i = 0; i < 3; ++i) opq[i] = operand(i);
    }
    // K(tau+2) and V(tau): 4-wave groups (four buffer loads each of K and V per wave) issue them
    // after the first MFMA slot, so that MFMA starts sooner after the barrier; 8-wave groups
    // (two each) at the step start (measured: C3 -2.4%, C2 unchanged or slower otherwise)
    constexpr int kLoadSlot = NW == 4 ? 1 : -1;
    // K(tau+kL+1) and V(tau+kL-1) (with two buffers: buffer cb, the literal)
    char* const kdst = kRing == 2 ? kb_lds(cb) : kb_lds(tau + kL + 1);
    char* const vdst = kRing == 2 ? vb_lds(cb) : vb_lds(tau + kL - 1);
    [[maybe_unused]] float ksc_n = 0.f, vsc_n = 0.f;  // fp8 pools: scales of the fetched tiles
    auto issue_loads = [&]() {
      if constexpr (PK) {
        if (tau + kL + 1 < ntau)
          loader.issue_k_packed(kpool, a.pool_bytes, kp.off + kp.t0 * (kHeadDim * 2),
                                kp.off_n - (a.T - kp.t0) * (kHeadDim * 2), a.T - kp.t0, kdst);
        if (tau + kL - 1 < ntau)
          loader.issue_v_packed(vpool, a.pool_bytes, vp.off + vp.t0 * 2, vp.off_n - (a.T - vp.t0) * 2,
                                a.T - vp.t0, vdst);
      } else if constexpr (kFp8Pool) {
        // codes and scales of K(tau+kL+1) and V(tau+kL-1) into registers now, decoded at the
        // step's end (the step's products cover the loads' latency)
        if (tau + kL + 1 < ntau) {
          loader.fetch_k(kpool + kw.base + (int64_t)kw.t * kTile * kHeadDim);
          ksc_n = a.kscale[(int64_t)kw.slot * n_bh + bh];
        }
        if (tau + kL - 1 < ntau) {
          loader.fetch_v(vpool + vw.base + vw.t * kTile);
          vsc_n = a.vscale[(int64_t)vw.slot * n_bh + bh];
        }
      } else {
        if (tau + kL + 1 < ntau) loader.issue_k(kpool + kw.base + (int64_t)kw.t * kTile * kHeadDim, kdst, w);
        if (tau + kL - 1 < ntau) loader.issue_v(vpool + vw.base + vw.t * kTile, vdst, w);
      }
    };
    if (kLoadSlot < 0) issue_loads();
    if constexpr (RM == 2) {
      // W for the frame tile tau+kL+1 opens (rot_q reads it at the start of step tau+kL)
      if (tau + kL + 1 < ntau && kw.t == 0) issue_w(kw.j);
    }
    if constexpr (RM > 0) {
      // QK(tau+1) below opens a new key frame: turn Q's temporal pairs for it
      if (tau + 1 < ntau && mw.t == 0) rot_q(mw.j);
    }
    if constexpr (RM == 2) {
#pragma unroll
      for (int i = 0; i < 3; ++i) opq[i] = operand(i);
    }

    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float ls[4];
    float pf[32];
    auto prob = [&](int e, float mu) {
      const float p = __builtin_amdgcn_exp2f(fmaf(s_cur[e >> 4][e & 15], c2, -mu));
      pf[e] = p;
      ls[e & 3] += p;
      if (e & 1) {
        pb[e >> 4][(e >> 3) & 1][(e & 7) - 1] = (ET)pf[e - 1];
        pb[e >> 4][(e >> 3) & 1][e & 7] = (ET)p;
      }
    };
    constexpr bool kFront = RM != 2;  // softmax schedule, below
    float lp, lp01, lp23;
    bool need;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (i + 3 < 32) opq[(i + 3) & 3] = operand(i + 3);
      if (i == kLoadSlot) issue_loads();
      // wave priority falls over the tile (2, 1, 0 by thirds): the wave that is ahead yields
      // issue slots to the one behind, so both reach the tile's barrier closer together
      if (i == 0) __builtin_amdgcn_s_setprio(2);
      if (i == 11) __builtin_amdgcn_s_setprio(1);
      if (i == 22) __builtin_amdgcn_s_setprio(0);
      const int st = i >> 1;
      if ((i & 1) == 0) {
        const int k = st >> 1, kbb = st & 1;
        s_nxt[kbb] = mfma32(opq[i & 3], qf[k], k == 0 ? zero16 : s_nxt[kbb]);
      } else {
        int db, kbb, s2;
        pv_order(st, db, kbb, s2);
        oacc[db] = mfma32(opq[i & 3], pprev[kbb][s2], oacc[db]);
      }
      // softmax of tile tau, front-loaded: slot i < 4 takes probabilities 2i and 2i+1, slot
      // 4 <= i < 28 probability i + 4; each is summed and packed one slot after its exp (so no
      // VALU op waits on the transcendental unit), and slots 29 and 30 form the row sum, so the
      // rare-path test after the last MFMA has its operands ready.  PRoPE keeps one probability
      // per slot (its frame-boundary query transform leaves no registers for the extra exps).
      {
        auto retire = [&](int d) {
          ls[d & 3] = d < 4 ? pf[d] : ls[d & 3] + pf[d];
          asm volatile("" ::"v"(ls[d & 3]));
          if (d & 1) {
            pb[d >> 4][(d >> 3) & 1][(d & 7) - 1] = (ET)pf[d - 1];
            pb[d >> 4][(d >> 3) & 1][d & 7] = (ET)pf[d];
          }
          if ((d & 7) == 7) asm volatile("" ::"v"(pb[d >> 4][(d >> 3) & 1]));
        };
        auto expo = [&](int e) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s_cur[e >> 4][e & 15], c2, -m_use));
          asm volatile("" ::"v"(p));  // keep this exp next to its MFMA
          pf[e] = p;
        };
        if constexpr (kFront) {
          if (i >= 1 && i <= 4) {
            retire(2 * (i - 1));
            retire(2 * (i - 1) + 1);
          } else if (i >= 5 && i <= 28) {
            retire(i + 3);
          }
          if (i < 4) {
            expo(2 * i);
            expo(2 * i + 1);
          } else if (i < 28) {
            expo(i + 4);
          }
          if (i == 29) {
            lp01 = ls[0] + ls[1];
            lp23 = ls[2] + ls[3];
          }
          if (i == 30) {
            lp = lp01 + lp23;
            need = !(lp <= kMaxPart) || m_run == -INFINITY;
          }
        } else {
          if (i > 0) retire(i - 1);
          expo(i);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!kFront) {
      ls[3] += pf[31];
      pb[1][1][6] = (ET)pf[30];
      pb[1][1][7] = (ET)pf[31];
      lp = (ls[0] + ls[1]) + (ls[2] + ls[3]);
      need = !(lp <= kMaxPart) || m_run == -INFINITY;
    }
    if (__any(need)) {
      // rare path: both key halves of a query take the same decision; raise the max of each
      // such query to the tile's true max, recompute its probabilities, rescale O and l
      const bool needq = pair_max(need ? 1.f : 0.f) > 0.f;
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 32; ++e) mx = fmaxf(mx, s_cur[e >> 4][e & 15]);
      mx = pair_max(mx) * c2;
      const float m_new = needq ? fmaxf(m_run, mx) : m_run;
      const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float mu = m_new == -INFINITY ? 0.f : m_new;  // = m_use for lanes kept
#pragma unroll
      for (int e = 0; e < 4; ++e) ls[e] = 0.f;
#pragma unroll
      for (int e = 0; e < 32; ++e) prob(e, mu);
      lp = (ls[0] + ls[1]) + (ls[2] + ls[3]);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
      m_run = m_new;
    }
    l_run += lp;
    if (tau + 1 < ntau) {
      if constexpr (PK) {
        const int key0 = (tb + tau + 1) * kTile;
        if (key0 + kTile > lim_lo) mask_tile(s_nxt, hh, 0, 1 << 30, key0, lim_lane);
      } else {
        int tok0, key0;
        if (walk_needs_mask(mw, tok0, key0)) mask_tile(s_nxt, hh, tok0, mw.flen, key0, lim_lane);
      }
    }
    if constexpr (PK) {
      kp.next(a, kbh);
      vp.next(a, kbh);
    } else {
      kw.next(a, kbh);
      vw.next(a, kbh);
      mw.next(a, kbh);
    }
    if constexpr (kFp8Pool) {
      // the codes fetched with the step's loads, decoded into buffers no wave reads this step
      if (tau + kL + 1 < ntau) loader.commit_k(kdst, w, ksc_n);
      if (tau + kL - 1 < ntau) loader.commit_v(vdst, w, vsc_n);
    }
    if (kL == 1 || cb == 1) {
      // the loads of the last kL steps have landed; every wave is done with the buffers the
      // next kL steps load into (read kL steps before those loads)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
  };
  static_assert(kL == 1 || kL == 2, "the barrier test above assumes kL <= 2 (cb = tau & 1)");
  int tau = 0;
  for (; tau + 1 < ntau; tau += 2) {
    step(tau, 0, sA, sB, pA, pB);
    step(tau + 1, 1, sB, sA, pB, pA);
  }
  // Epilogue: PV(ntau-1); V(ntau-1) was loaded kL steps earlier (or by the prologue), with a
  // barrier in between.
  auto epilogue = [&](const etx8 (&pprev)[2][2]) __attribute__((always_inline)) {
    const char* vl = vb_lds(ntau - 1) + lane16;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int kbb = 0; kbb < 2; ++kbb)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const etx8 av =
              *reinterpret_cast<const etx8*>(vl + (db * 4 + kbb * 2 + s2) * kBlockBytes);
          oacc[db] = mfma32(av, pprev[kbb][s2], oacc[db]);
        }
  };
  if (tau < ntau) {
    step(tau, 0, sA, sB, pA, pB);
    epilogue(pB);
  } else if (ntau > 0) {
    epilogue(pA);
  }

  const float l_tot = pair_sum(l_run);
  if (SPLIT && (tb > 0 || te < nt)) {
    // part of a split q-tile: unnormalised O, the running max and the row sum
    if (qlive) {
      const int64_t row = (2 * (int64_t)logical + (seg > 0 ? 1 : 0)) * kBQ + w * 32 + n;
      float* po = a.part_o + row * kHeadDim;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(po + db * 32 + g * 8 + hh * 4) =
              f32x4{oacc[db][g * 4], oacc[db][g * 4 + 1], oacc[db][g * 4 + 2], oacc[db][g * 4 + 3]};
      if (hh == 0) *reinterpret_cast<float2*>(a.part_ml + row * 2) = make_float2(m_run, l_tot);
    }
    continue;
  }
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (qlive) {
    QT* op = static_cast<QT*>(a.o) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
             (int64_t)qrow * a.o_st;
    // lane (n, hh) holds channels db*32 + g*8 + hh*4 .. +3 of its query: whole PRoPE groups
    [[maybe_unused]] const float* po = nullptr;
    if constexpr (RM == 2) po = a.pq_o + ((int64_t)b * a.n_qframes + qfi) * 16;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + g * 8 + hh * 4;
        float x0 = oacc[db][g * 4 + 0] * inv, x1 = oacc[db][g * 4 + 1] * inv;
        float x2 = oacc[db][g * 4 + 2] * inv, x3 = oacc[db][g * 4 + 3] * inv;
        if constexpr (RM == 2) {
          const float y0 = fmaf(po[0], x0, fmaf(po[1], x1, fmaf(po[2], x2, po[3] * x3)));
          const float y1 = fmaf(po[4], x0, fmaf(po[5], x1, fmaf(po[6], x2, po[7] * x3)));
          const float y2 = fmaf(po[8], x0, fmaf(po[9], x1, fmaf(po[10], x2, po[11] * x3)));
          const float y3 = fmaf(po[12], x0, fmaf(po[13], x1, fmaf(po[14], x2, po[15] * x3)));
          x0 = y0, x1 = y1, x2 = y2, x3 = y3;
        }
        store4<QT>(op + d0, x0, x1, x2, x3);
      }
  }
  }  // segments
}

// ---------------------------------------------------------------------------------------------
// fp8-e4m3 pools (one dequantisation scale per (slot, stream, head) for K and for V), on gfx950's
// v_mfma_f32_32x32x64_f8f6f4: each operand lane (n, hh) holds row / column n and k values
// 32 hh .. 32 hh + 31 (32 bytes).
//   * Q is quantised in-kernel per query row (scale = absmax/448); the K frame scale and the Q
//     row scale fold into the softmax FMA: x = acc * (log2e*scale*sq*sk) - m;
//   * P is quantised as P * sv * G (sv = the tile's V frame scale, G = 28 / max_window(sv), so
//     P <= 16 maps below 448) and O is divided by G * sum(P) at the end;
//   * the running max is speculative, as in attn_kernel: probabilities are formed against the
//     max of the earlier tiles.  The row sums of the stored P come from the matrix core (one
//     16x16x128 product per tile, mfma_rowsum) instead of 32 VALU adds per lane; a stored
//     probability that does not fit e4m3 (>= 480) converts to NaN, so a NaN row sum, or a max
//     still -inf, sends the wave to a rare path that raises the max to the tile's true max and
//     recomputes the tile.  The test runs at the start of the next step, before that tile's
//     PV product and before its scores' registers take the next QK product (P up to 16 x the
//     row max's fits without it);
//   * per 64-key tile and wave: 4 QK MFMAs (2 key blocks kb x 2 channel halves cs; A = K rows,
//     B = the lane's 32 quantised Q channels cs*64 + 32 hh ..) and 4 PV MFMAs (one per
//     32-channel block db; A = V^T row 32 db + n, keys 32 hh .. +31; B = P^T, the lane's
//     probabilities of keys 32 hh .. +31 in key order);
//   * K rows are staged in the order key_perm64(kb, r), which puts key 32 hh + 16 kb + i of the
//     tile in accumulator register i of lane half hh, so the scores of a lane are already in
//     P^T's operand order;
//   * LDS: one 2 KB operand block per (kb, cs) for K and per db for V^T, stored as two 1 KB
//     halves: half q holds bytes 16 q .. +16 of every operand lane, lane L at 16 L.  Both
//     ds_read_b128 of an operand then read 64 consecutive 16 B pieces (no bank conflicts; a
//     lane-contiguous 32 B layout costs a 2-way conflict on every read).  Direct buffer->LDS
//     loads fill them: DMA lane i of part q writes operand lane i, bytes 16 q .. +16.
constexpr int kOp8 = 2048;
// K and V^T tile buffers of the fp8 kernel's ring: a barrier every ring / 2 steps (8 measured
// slower than 4 at C5: the waves drift further apart between barriers).  4-wave groups keep two
// buffers (with four they spill a register).
constexpr int fp8_ring(int nw) { return nw == 8 ? 4 : 2; }
// dynamic LDS of attn_fp8_kernel: the K and V^T rings (4 operand blocks of kOp8 bytes per tile);
// for RoPE on load (RM = 1) also each wave's 4 KB of query channels 0..63 in bf16 (the temporal
// pairs unrotated), from which the temporal part of the fp8 query is rebuilt per key frame, and
// one table slot per ring buffer: the temporal angles (22 pairs x cos, sin = 176 B) of the
// q-tile's query frames (at most 5) against the key frame a tile opens
constexpr int kFp8QRows = 4096;
constexpr int kFp8TabSlot = 1024;
constexpr int kFp8TabFrames = 5;
static_assert(kFp8TabFrames * 8 * kRopeT <= kFp8TabSlot && kFp8TabFrames * 11 <= 64,
              "one 64-lane DMA of 16 B pieces fills a table slot");
static_assert((256 - 1) / 64 + 2 <= kFp8TabFrames, "256 rows of >= 64-token frames span <= 5 frames");
constexpr int fp8_lds_bytes(int nw, int rm = 0) {
  return 2 * fp8_ring(nw) * 4 * kOp8 +
         (rm == 1 ? nw * kFp8QRows + fp8_ring(nw) * kFp8TabSlot : 0);
}
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ inline int key_perm64(int kb, int r) {
  return 32 * ((r >> 2) & 1) + 16 * kb + 4 * (r >> 3) + (r & 3);
}

// QK step t of a tile -> K operand block c = 2 kb + cs: (0,0), (1,0), (0,1), (1,1)
__device__ inline int korder64(int t) { return ((t & 1) << 1) | (t >> 1); }

__device__ inline int pack_fp8x4(float x0, float x1, float x2, float x3) {
  const int v = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, v, true);
}
// The same into a register whose previous contents are overwritten whole by the two converts
// (low then high half), so no zeroing move is needed.
__device__ inline int pack_fp8x4_into(int old, float x0, float x1, float x2, float x3) {
  const int v = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, old, false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, v, true);
}

__device__ inline void mask_tile64(f32x16 (&s)[2], int hh, int tok0, int T, int key0, int lim) {
  // as mask_tile: key kk = 32 hh + 16 kb + i is masked when kk >= min(T - tok0, lim - key0)
  const int t = min(T - tok0, lim - key0) - 32 * hh;
  mask_regs<KeyFp8>(s, t, std::make_integer_sequence<int, 32>{});
}

// the lane's 32-byte operand: p = block + 16 * lane (first half), second half 1 KB further
__device__ inline i32x8 lds_op32(const char* p) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
  const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 1024);
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
               (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// max(a, b, c) without the IEEE quieting of the inputs (no input is a signalling NaN)
__device__ inline float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ inline float pair_max_raw(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max3_raw(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[1]));
}

__device__ inline f32x16 mfma64(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// Row sums of P on the matrix core: the 32x32x64 B operand P^T (lane (n, hh) = query n, keys
// 32 hh ..) read as the B operand of the 16x16x128 product is column n & 15 with K group
// (n >> 4) + 2 hh; A row r is 1.0 (e4m3 0x38) on the K groups of parity (r >> 2) & 1 and 0
// elsewhere, so output rows 4g .. 4g+3 (held by lanes 16g ..) sum query (n & 15) + 16 (g & 1)
// over both key halves: every lane receives its own query's sum.
__device__ inline f32x4 mfma_rowsum(const i32x8& ones, const i32x8& p, const f32x4& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ones, p, c, 0, 0, 0, 0, 0, 0);
}

// direct buffer->LDS copy of this lane's N 16-byte pieces of one tile: goff = the piece's byte
// offset inside the tile, loff = its byte offset inside the LDS buffer
template <int N>
struct Stage64 {
  uint32_t goff[N];
  int loff[N];
  __device__ void operator()(const uint8_t* tile, char* buf) const {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass would drop the calling kernels' launch stubs
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)tile, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int j = 0; j < N; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(buf + loff[j]), 16, goff[j], 0, 0, 0);
#endif
  }
};

// scores of one 64-key tile: s[kb] = K rows (kb, both channel halves) . Q
__device__ inline void qk64(const char* kl, const i32x8 (&q8)[2], const f32x16& zero16,
                            f32x16 (&s)[2]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    s[kb] = mfma64(lds_op32(kl + (kb * 2) * kOp8), q8[0], zero16);
    s[kb] = mfma64(lds_op32(kl + (kb * 2 + 1) * kOp8), q8[1], s[kb]);
  }
}

// RM = 1: RoPE on load (the K pool is the fp8 copy with its height/width pairs rotated, the
// temporal pairs raw).  The query's height/width pairs are rotated once at load; its temporal
// pairs (channels 0..43, which lie in the lane's first 32-channel slice) are turned by the angle
// of (query frame, key frame) and quantised again whenever the key walk enters a frame.  The
// row scale bounds every rotation: max(spatial |q|, temporal pair norms) / 448.
template <int NW, typename QT, bool SPLIT = false, int RM = 0>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_fp8_kernel(AttnArgs a) {
  static_assert(RM == 0 || RM == 1, "fp8 MFMA attention: no RoPE or RoPE on load");
  constexpr int kBQ = NW * 32;
  constexpr int kDma = 16 / NW;     // 1 KB DMA parts per wave per tile (8 for K, 8 for V^T)
  constexpr int kBuf = 4 * kOp8;    // one K (or V^T) tile
  extern __shared__ __attribute__((aligned(16))) char lds[];
  int logical;
  {
    const int bid = blockIdx.x, xcd = bid & 7, idx = bid >> 3;
    const int per = a.n_wg >> 3, rem = a.n_wg & 7;
    logical = xcd * per + min(xcd, rem) + idx;
  }
  // Segments: key tiles [tb, te) of q-tile qg, as in attn_kernel (one whole q-tile unless split;
  // a split share runs its whole q-tiles, then its last segment, then its first).
  const int nt = a.nt;
  int q_first = logical, nseg = 1;
  int64_t u0 = 0, u1 = 0;
  if constexpr (SPLIT) {
    u0 = (int64_t)logical * a.units / a.n_wg;
    u1 = (int64_t)(logical + 1) * a.units / a.n_wg;
    q_first = (int)(u0 / nt);
    nseg = u1 > u0 ? (int)((u1 - 1) / nt) - q_first + 1 : 0;
  }
  for (int k = 0; k < nseg; ++k) {
  const int seg = nseg == 1 ? 0 : k < nseg - 2 ? k + 1 : k == nseg - 2 ? nseg - 1 : 0;
  const int qg = q_first + seg;
  int tb = 0, te = nt;
  if constexpr (SPLIT) {
    if (seg == 0) tb = (int)(u0 - (int64_t)q_first * nt);
    if (seg == nseg - 1) te = (int)(u1 - (int64_t)qg * nt);
  }
  if (k > 0) __syncthreads();  // the previous segment's last LDS reads are done
  const int qt = (qg + a.qt_base) % a.n_qtiles;
  const int bh = (qg + a.qt_base) / a.n_qtiles;
  const int h = bh % a.H, b = bh / a.H;
  // SPLIT: an opaque copy per segment keeps lane-derived values out of the segment loop's
  // live range
  int tid = threadIdx.x;
  if constexpr (SPLIT) asm volatile("" : "+v"(tid));
  const int lane = tid & 63, w = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int q0 = qt * kBQ;
  const int qrow = q0 + w * 32 + n;
  const bool qlive = qrow < a.Lq;

  // Q row quantisation: lane (n, hh) holds channels cs*64 + 32 hh .. +31 for cs = 0, 1.
  i32x8 q8[2];
  float q_scale;
  [[maybe_unused]] int qfi = 0;        // RM = 1: query frame of this lane's row
  [[maybe_unused]] float q_inv = 0.f;  // RM = 1: 448 / the row's bound
  {
    float qv[64];  // qv[cs * 32 + j] = channel cs * 64 + 32 hh + j
    const QT* qp = static_cast<const QT*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                   (int64_t)(qlive ? qrow : 0) * a.q_st + hh * 32;
    const float qn = a.q_rms && qlive ? a.q_rms[(int64_t)b * a.q_rms_sb + qrow] : 0.f;
    const float* qw = a.q_w + h * kHeadDim + hh * 32;
#pragma unroll
    for (int cs = 0; cs < 2; ++cs)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        Vec8<QT> v = qlive ? Vec8<QT>::load(qp + cs * 64 + c * 8) : Vec8<QT>::zero();
        if (a.q_rms) {  // normalised Q in bf16, as the reference's norm_q output
#pragma unroll
          for (int j = 0; j < 8; ++j)
            qv[cs * 32 + c * 8 + j] = (float)(bf16)((float)v.get(j) * qn * qw[cs * 64 + c * 8 + j]);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) qv[cs * 32 + c * 8 + j] = (float)(bf16)v.get(j);  // bf16 first
        }
      }
    float amax = 0.f;
    if constexpr (RM == 1) {
      // height/width pairs (global pair index cs * 32 + 16 hh + m >= 22) turned by the query's
      // own position, in fp32 from the values above, then rounded to bf16 (the roped bf16
      // query); temporal pairs stay as loaded and bound the scale by their norms.  Every product
      // and sum rounds on its own (no contraction), so the fp8 codes are a fixed function of the
      // inputs that a CPU restatement reproduces exactly.
#pragma clang fp contract(off)
      const int qr = qlive ? qrow : a.Lq - 1;
      qfi = qr / a.T;
      const int tt = qr - qfi * a.T, hq = tt / a.gw, wq = tt - hq * a.gw;
      // every lane loads an in-bounds table entry and selects (no lane-divergent branches)
#pragma unroll
      for (int cs = 0; cs < 2; ++cs)
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          const int pr = cs * 32 + hh * 16 + m;
          const bool temporal = pr < kRopeT;
          float& u = qv[cs * 32 + 2 * m];
          float& v = qv[cs * 32 + 2 * m + 1];
          const int idx = pr < kRopeT + kRopeHW ? hq * kRopeHW + max(pr - kRopeT, 0)
                                                : (a.gh + wq) * kRopeHW + (pr - kRopeT - kRopeHW);
          const float2 cn = *reinterpret_cast<const float2*>(a.rope_hw + 2 * idx);
          const float u2 = (float)(bf16)(u * cn.x - v * cn.y), v2 = (float)(bf16)(u * cn.y + v * cn.x);
          const float bound = temporal ? __builtin_sqrtf(u * u + v * v)
                                       : fmaxf(__builtin_fabsf(u2), __builtin_fabsf(v2));
          amax = fmaxf(amax, bound);
          u = temporal ? u : u2;
          v = temporal ? v : v2;
        }
      // slice 0 (channels 32 hh .. +31) to this wave's LDS rows: chunk c of lane L at c KB + 16 L
      char* qs = lds + fp8_lds_bytes(NW) + w * kFp8QRows + lane * 16;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        bf16x8 t;
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] = (bf16)qv[8 * c + e];
        *reinterpret_cast<bf16x8*>(qs + c * 1024) = t;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 64; ++j) amax = fmaxf(amax, __builtin_fabsf(qv[j]));
    }
    amax = pair_max(amax);
    const float inv = amax > 0.f ? 448.0f / amax : 0.f;
    q_scale = amax / 448.0f;
    q_inv = inv;
    auto cl = [&](float x) { return fminf(fmaxf(x * inv, -448.f), 448.f); };
#pragma unroll
    for (int cs = 0; cs < 2; ++cs)
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const float* t = qv + cs * 32 + 4 * d;
        q8[cs][d] = pack_fp8x4(cl(t[0]), cl(t[1]), cl(t[2]), cl(t[3]));
      }
  }

  const int n_keys = (int)a.n_keys;
  int lim_lane = n_keys, lim_lo = n_keys, lim_hi = n_keys;
  if (a.mask_mode == SKV_MASK_CHUNK_CAUSAL) {
    const int qlast = min(q0 + kBQ, a.Lq) - 1;
    lim_lane = (int)chunk_limit(a.q_pos0 + min(qrow, a.Lq - 1), a.chunk, n_keys);
    lim_lo = (int)chunk_limit(a.q_pos0 + q0, a.chunk, n_keys);
    lim_hi = (int)chunk_limit(a.q_pos0 + qlast, a.chunk, n_keys);
  }
  int ntau;
  {
    const int jf = lim_hi / a.T;
    ntau = jf >= a.n_frames ? a.n_frames * a.ntiles_f
                            : jf * a.ntiles_f + (lim_hi - jf * a.T + kTile - 1) / kTile;
    if constexpr (SPLIT) ntau = te - tb;  // no mask: the segment's tiles
  }

  const uint8_t* kpool = static_cast<const uint8_t*>(a.kpool);
  const uint8_t* vpool = static_cast<const uint8_t*>(a.vpool);
  const int64_t kbh = (int64_t)(b * a.H + h) * a.Tp * kHeadDim;
  const int64_t sc_bh = (int64_t)b * a.H + h;
  auto ktile = [&](int tau) {  // tile tau of the segment
    const int x = tb + tau, j = x / a.ntiles_f, t = x - j * a.ntiles_f;
    return kpool + (int64_t)a.slots[j] * a.slot_stride + kbh + (int64_t)t * kTile * kHeadDim;
  };
  auto tile_needs_mask = [&](int tau, int& tok0, int& key0, int& tj) -> bool {
    const int x = tb + tau, j = x / a.ntiles_f, t = x - j * a.ntiles_f;
    tok0 = t * kTile;
    key0 = j * a.T + tok0;
    tj = a.flen[j];
    return (tok0 + kTile > tj) || (key0 + kTile > lim_lo);
  };
  // staging: wave wu moves parts c = wu * kDma + j; parts 0..7 are K (block c >> 1 = (kb, cs),
  // half c & 1), parts 8..15 V^T (block db = (c - 8) >> 1, half c & 1); a wave is all K or all V
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const bool kload = wu * kDma < 8;
  Stage64<kDma> stage;
#pragma unroll
  for (int j = 0; j < kDma; ++j) {
    const int c = wu * kDma + j, p = c & 1;
    if (c < 8) {  // operand lane `lane` = (row n, channels cs*64 + 32 hh ..), bytes 16 p ..
      const int blk = c >> 1;
      stage.goff[j] = (uint32_t)(key_perm64(blk >> 1, lane & 31) * kHeadDim + (blk & 1) * 64 +
                                 32 * (lane >> 5) + 16 * p);
      stage.loff[j] = blk * kOp8 + p * 1024;
    } else {  // operand lane `lane` = (channel 32 db + n, keys 32 hh ..), bytes 16 p ..
      const int db = (c - 8) >> 1;
      stage.goff[j] = (uint32_t)((32 * db + (lane & 31)) * a.Tp + 32 * (lane >> 5) + 16 * p);
      stage.loff[j] = db * kOp8 + p * 1024;
    }
  }
  // K and V^T tiles each cycle through kRing LDS buffers (tile x in buffer x mod kRing): a step
  // reads K(tau+1) and V(tau-1) and loads K(tau+3) and V(tau+1), so the buffers a step writes
  // were last read two steps earlier, and the workgroup meets at a barrier after every second
  // step (odd tau) only.
  constexpr int kRing = fp8_ring(NW);
  constexpr int kL = kRing / 2;  // steps between barriers
  auto kb_lds = [&](int i) { return lds + (i & (kRing - 1)) * kBuf; };
  auto vb_lds = [&](int i) { return lds + (kRing + (i & (kRing - 1))) * kBuf; };

  // RM = 1: the temporal angles of the q-tile's query frames qf_lo .. (at most kFp8TabFrames,
  // checked by the host) against key frame j -> the table slot of the tile x that opens frame j
  // (slot x mod kRing, written with K(x) and read before QK(x), so it lives like K(x)'s buffer).
  // Lane i moves 16 bytes: pairs 2 (i % 11) .. +1 of query frame qf_lo + i / 11; lanes past the
  // q-tile's frames repeat frame qf_lo's pieces into the slot's unread tail.
  [[maybe_unused]] const int qf_lo = q0 / a.T;
  [[maybe_unused]] char* const tab_lds = lds + fp8_lds_bytes(NW) + NW * kFp8QRows;
  [[maybe_unused]] auto stage_tab = [&](int x, int j) __attribute__((always_inline)) {
    if constexpr (RM == 1) {
      const int count = (min(q0 + kBQ, a.Lq) - 1) / a.T - qf_lo + 1;
      const int f = lane / 11, pp = lane - 11 * f;
      Stage64<1> st;
      st.goff[0] = (uint32_t)((((qf_lo + (f < count ? f : 0)) * a.n_frames + j) * kRopeT + 2 * pp) * 8);
      st.loff[0] = (x & (kRing - 1)) * kFp8TabSlot;
      st(reinterpret_cast<const uint8_t*>(a.rope_t), tab_lds);
    }
  };
  // RM = 1: q8[0] (channels 32 hh .. +31) rebuilt for the key frame tile x opens: the temporal
  // pairs (global index 16 hh + 4 c + m < 22) turned by the angle of (this row's query frame,
  // that key frame) in fp32, rounded to bf16 and quantised with the row's scale; the other pairs
  // of the slice (roped at load) take an exact identity turn and quantise as before.  Every lane
  // reads an in-bounds table entry and selects.
  [[maybe_unused]] auto requant = [&](int x) __attribute__((always_inline)) {
    if constexpr (RM == 1) {
#pragma clang fp contract(off)
      // pairs 16 hh .. +15 of the row's query frame (128 B from a 32-aligned offset inside the
      // slot: (qfi - qf_lo) * 176 + 128 hh + 128 <= 4 * 176 + 256 < kFp8TabSlot), 4 pairs per
      // chunk c read by an asm block: the compiler's own LDS reads of a DMA-written buffer would
      // first wait for every DMA in flight (the next tiles' K and V), which the barrier after the
      // slot's DMA already covers
      const uint32_t tab = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(
          tab_lds + (x & (kRing - 1)) * kFp8TabSlot + (qfi - qf_lo) * (8 * kRopeT) + hh * 128);
      const char* qs = lds + fp8_lds_bytes(NW) + w * kFp8QRows + lane * 16;
      auto cl = [&](float v) { return fminf(fmaxf(v * q_inv, -448.f), 448.f); };
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        f32x4 tq[2];  // cos, sin of pairs 16 hh + 4 c .. +1, then +2 .. +3
        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(tq[0]), "=&v"(tq[1])
                     : "v"(tab + 32 * c));
        const bf16x8 t = *reinterpret_cast<const bf16x8*>(qs + c * 1024);
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = (float)t[e];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          // pair 16 hh + 4 c + m: temporal below 22; the others read past the frame's 22 pairs
          // (values discarded by the select)
          const bool temporal = hh * 16 + c * 4 + m < kRopeT;
          const float cr = temporal ? tq[m >> 1][2 * (m & 1)] : 1.0f;
          const float sr = temporal ? tq[m >> 1][2 * (m & 1) + 1] : 0.0f;
          const float u = y[2 * m], v = y[2 * m + 1];
          y[2 * m] = (float)(bf16)(u * cr - v * sr);
          y[2 * m + 1] = (float)(bf16)(u * sr + v * cr);
        }
        q8[0][2 * c] = pack_fp8x4(cl(y[0]), cl(y[1]), cl(y[2]), cl(y[3]));
        q8[0][2 * c + 1] = pack_fp8x4(cl(y[4]), cl(y[5]), cl(y[6]), cl(y[7]));
      }
    }
  };

  float sv_max = 0.f;
  for (int j = 0; j < a.n_frames; ++j)
    sv_max = fmaxf(sv_max, a.vscale[(int64_t)a.slots[j] * a.B * a.H + sc_bh]);
  const float G = sv_max > 0.f ? 28.0f / sv_max : 1.0f;
  const float c2q = a.scale_log2 * q_scale;
  const int lane16 = lane * 16;

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  // A operand of the row-sum product (mfma_rowsum)
  i32x8 ones;
  {
    const int v = (((lane >> 4) ^ (lane >> 2)) & 1) ? 0 : 0x38383838;
#pragma unroll
    for (int i = 0; i < 8; ++i) ones[i] = v;
  }
  f32x4 tsum;  // row sums of the last tile's stored P, from the matrix core
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  f32x16 zero16;
#pragma unroll
  for (int i = 0; i < 16; ++i) zero16[i] = 0.f;

  // score and probability registers ping-pong between two sets (A, B) across iterations (the
  // loop is unrolled twice), so no loop-carried copy is needed
  f32x16 sA[2], sB[2];
  i32x8 pA = {0, 0, 0, 0, 0, 0, 0, 0}, pB;
  // Prologue: K(0), K(1), K(2) and V(0) resident, V(-1)'s buffer zeroed so PV(-1) of step 0 adds
  // nothing; then QK(0).
  TileWalk<> w0;  // tile 0 of the segment: V(0) and the scales of its frame
  w0.start(a, kbh, tb);
  if (ntau > 0) {
#pragma unroll
    for (int x = 0; x <= kL; ++x)
      if (x < ntau) if (kload) stage(ktile(x), kb_lds(x));
    if (!kload) {
      TileWalk<> wv = w0;
#pragma unroll
      for (int x = 0; x < kL - 1; ++x) {
        if (x < ntau) stage(vpool + wv.base + wv.t * kTile, vb_lds(x));
        wv.next(a, kbh);
      }
    }
    if constexpr (RM == 1) {  // the angles for tile 0's frame and for frames tiles 1..kL open
      if (wu == 0) {
        stage_tab(0, w0.j);
#pragma unroll
        for (int x = 1; x <= kL; ++x) {
          const int g = tb + x, j = g / a.ntiles_f;
          if (x < ntau && g == j * a.ntiles_f) stage_tab(x, j);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 8 / NW; ++r)
      *reinterpret_cast<u32x4*>(vb_lds(-1) + (tid + NW * 64 * r) * 16) = u32x4{0u, 0u, 0u, 0u};
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if constexpr (RM == 1) requant(0);  // the query for the frame of tile 0
    qk64(kb_lds(0) + lane16, q8, zero16, sA);
    int tok0, key0, tj;
    if (tile_needs_mask(0, tok0, key0, tj)) mask_tile64(sA, hh, tok0, tj, key0, lim_lane);
    __syncthreads();  // K(0) read by every wave before its buffer takes K(4)
  }
  // Tiles addressed in step tau: K(tau+3) (kw), V(tau+1) (vw), the mask and the scales of
  // tile tau+1 (mw); the walks advance one tile per step.
  TileWalk<> kw, vw, mw;
  kw.start(a, kbh, tb + kL + 1);
  vw.start(a, kbh, tb + kL - 1);
  mw.start(a, kbh, tb + 1);
  // Per key frame: the softmax multiplier (K scale folded in) and the log and reciprocal of the
  // P scale, for the frame of the tile whose softmax runs next.
  float mult = 0.f, log_pv = 0.f, inv_pv = 1.0f;
  auto open_scales = [&](int slot) {
    const int64_t sc = (int64_t)slot * a.B * a.H + sc_bh;
    // an all-zero query row or K frame makes every logit 0; keep the multiplier positive so
    // masked (-inf) logits stay -inf instead of becoming NaN.  The scales are read through the
    // constant address space (scalar loads).
    typedef const __attribute__((address_space(4))) float* cfloat_p;
    mult = fmaxf(c2q * ((cfloat_p)(uintptr_t)a.kscale)[sc], 1e-30f);
    // P is stored as p * sv * G: the factor rides in the exponent's bias (one log per key frame
    // instead of 32 multiplies per tile) and the row sum divides it out once.  An all-zero V
    // frame (sv = 0) keeps P unscaled: its V codes are all 0, so only the sum sees P.
    const float pv_raw = ((cfloat_p)(uintptr_t)a.vscale)[sc] * G;
    const float pv = pv_raw > 0.f ? pv_raw : 1.0f;
    log_pv = __builtin_amdgcn_logf(pv);
    inv_pv = __builtin_amdgcn_rcpf(pv);
  };
  if (ntau > 0) open_scales(w0.slot);
  int open_slot = -1;  // the slot of the frame the next tile opens (wave-uniform), else -1
  // Settles P of the previous tile (scores s) before its PV product.  Probabilities use the
  // running max m, not the tile's own max: an e4m3 probability at or above 480 converts to NaN,
  // so its query's row sum from the matrix core is NaN, and that (or m still -inf) sends the
  // wave to the rare path, which raises m of such queries to the tile's true max, recomputes
  // their probabilities and rescales O and l.  The scales are still those of that tile's frame.
  // rare path for P of one tile (scores s, packs p, lane decision `need`)
  auto rare = [&](const f32x16 (&s)[2], i32x8& p, bool need) __attribute__((always_inline)) {
    {
      // both key halves of a query take the same decision
      const bool needq = pair_max(need ? 1.f : 0.f) > 0.f;
      float mq[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const f32x16& sc = s[c];
        mq[c] = max3_raw(sc[0], sc[1], sc[2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) mq[c] = max3_raw(mq[c], sc[r], sc[r + 1]);
        mq[c] = max3_raw(mq[c], sc[15], sc[15]);
      }
      const float mx = pair_max_raw(max3_raw(mq[0], mq[1], mq[1])) * mult;
      const float m_new = needq ? fmaxf(m_run, mx) : m_run;
      const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float bias2 = log_pv - (m_new == -INFINITY ? 0.f : m_new);
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        float q4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int e = 4 * d + j;
          q4[j] = __builtin_amdgcn_exp2f(fmaf(s[e >> 4][e & 15], mult, bias2));
        }
        p[d] = pack_fp8x4_into(p[d], q4[0], q4[1], q4[2], q4[3]);
      }
      tsum = mfma_rowsum(ones, p, zero4);
      l_run *= alpha;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
      }
      m_run = m_new;
    }
  };
  auto settle = [&](const f32x16 (&s)[2], i32x8& p) __attribute__((always_inline)) {
    const bool need = !(tsum[0] <= 3.0e38f) || m_run == -INFINITY;
    if (__any(need)) rare(s, p, need);
    l_run = fmaf(tsum[0], inv_pv, l_run);
  };
  // cb = tau & 1, passed as a literal: the register sets alternate with it, and odd steps end
  // at the barrier
  auto step = [&](int tau, const int cb, f32x16 (&s_cur)[2], f32x16 (&s_nxt)[2], i32x8& pprev,
                  i32x8& pb) __attribute__((always_inline)) {
    if (tau + kL + 1 < ntau) {
      if (kload) stage(kpool + kw.base + (int64_t)kw.t * kTile * kHeadDim, kb_lds(tau + kL + 1));
      if constexpr (RM == 1)  // tile tau+kL+1 opens frame kw.j: its angles travel with K
        if (wu == 0 && kw.t == 0) stage_tab(tau + kL + 1, kw.j);
    }
    if (tau + kL - 1 < ntau) if (!kload) stage(vpool + vw.base + vw.t * kTile, vb_lds(tau + kL - 1));
    if (tau > 0) settle(s_nxt, pprev);  // s_nxt still holds the scores of tile tau-1
    if (open_slot >= 0) {  // tile tau opens a key frame
      open_scales(open_slot);
      open_slot = -1;
    }
    if constexpr (RM == 1)  // QK(tau+1) below takes the query of tile tau+1's frame
      if (tau + 1 < ntau && mw.t == 0) requant(tau + 1);
    const char* kl = kb_lds(tau + 1) + lane16;  // K(tau+1) (stale data on the last step)
    const char* vl = vb_lds(tau - 1) + lane16;  // V(tau-1) (zeros on the first step)

    // Eight MFMA slots, QK(tau+1) and PV(tau-1) alternating (QK steps in the order (kb, cs) =
    // (0,0), (1,0), (0,1), (1,1), so the two halves of one key block are four slots apart), each
    // followed by a quarter of softmax(tau): the 4 probabilities of P^T dword i.  The operands
    // come from LDS three slots ahead; the fp8 pack of a quarter runs one slot later, when its
    // exps have finished.
    i32x8 op[4];
    float pf[32];
    const float bias = log_pv - (m_run == -INFINITY ? 0.f : m_run);
#pragma unroll
    for (int i = 0; i < 3; ++i)
      op[i] = (i & 1) ? lds_op32(vl + (i >> 1) * kOp8) : lds_op32(kl + korder64(i >> 1) * kOp8);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i + 3 < 8) {
        const int j = i + 3;
        op[j & 3] = (j & 1) ? lds_op32(vl + (j >> 1) * kOp8) : lds_op32(kl + korder64(j >> 1) * kOp8);
      }
      if ((i & 1) == 0) {
        const int c = korder64(i >> 1), kb = c >> 1, cs = c & 1;
        s_nxt[kb] = mfma64(op[i & 3], q8[cs], cs == 0 ? zero16 : s_nxt[kb]);
      } else {
        oacc[i >> 1] = mfma64(op[i & 3], pprev, oacc[i >> 1]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * i + j;
        pf[e] = __builtin_amdgcn_exp2f(fmaf(s_cur[e >> 4][e & 15], mult, bias));
        asm volatile("" ::"v"(pf[e]));  // keep this quarter's exps next to its MFMA
      }
      if (i > 0) {
        const int d = i - 1;
        pb[d] = pack_fp8x4_into(pb[d], pf[4 * d], pf[4 * d + 1], pf[4 * d + 2], pf[4 * d + 3]);
        asm volatile("" ::"v"(pb[d]));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    pb[7] = pack_fp8x4_into(pb[7], pf[28], pf[29], pf[30], pf[31]);
    tsum = mfma_rowsum(ones, pb, zero4);  // read by the next step's settle
    if (tau + 1 < ntau) {
      const int tok0 = mw.t * kTile, key0 = mw.j * a.T + tok0;
      if ((tok0 + kTile > mw.flen) || (key0 + kTile > lim_lo))
        mask_tile64(s_nxt, hh, tok0, mw.flen, key0, lim_lane);
      if (mw.t == 0) open_slot = mw.slot;
    }
    kw.next(a, kbh);
    vw.next(a, kbh);
    mw.next(a, kbh);
    if (kL == 2 ? cb == 1 : (tau & (kL - 1)) == kL - 1) {
      // K(tau+2), K(tau+3), V(tau), V(tau+1) have landed; every wave is done with the buffers
      // the next two steps load into
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
  };
  int tau = 0;
  for (; tau + 1 < ntau; tau += 2) {
    step(tau, 0, sA, sB, pA, pB);
    step(tau + 1, 1, sB, sA, pB, pA);
  }
  // PV(ntau-1): V(ntau-1) was loaded by step ntau-2 (the prologue when ntau = 1), two steps or
  // a barrier earlier
  auto epilogue = [&](const f32x16 (&s_last)[2], i32x8& pprev) __attribute__((always_inline)) {
    // The last row-sum product (8 passes) was issued at the end of the step just before, and a
    // VALU read of its result must trail it by 12 wait states.  When the step skips its mask
    // block, the branch around that block can put settle's first read of tsum 2 issue slots
    // after the product (hipcc's own hazard pass has been seen to leave that path short, so a
    // lane read the previous tile's sum, skipped the rare path and summed NaN probabilities).
    // The wait is spelled out here, tied to tsum so that no read of it moves above it.
    asm volatile("s_nop 7\n\ts_nop 4" : "+v"(tsum));
    settle(s_last, pprev);
    const char* vl = vb_lds(ntau - 1) + lane16;
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] = mfma64(lds_op32(vl + db * kOp8), pprev, oacc[db]);
  };
  if (tau < ntau) {
    step(tau, 0, sA, sB, pA, pB);
    epilogue(sA, pB);
  } else if (ntau > 0) {
    epilogue(sB, pA);
  }
  // the matrix core sums both key halves of a query: every lane holds its query's full sum
  const float l_tot = l_run;
  if (SPLIT && (tb > 0 || te < nt)) {
    // part of a split q-tile: O / G (the P scale's G divided out), the running max in log2
    // units and the row sum, the record attn_combine_kernel merges
    if (qlive) {
      const float ig = 1.0f / G;
      const int64_t row = (2 * (int64_t)logical + (seg > 0 ? 1 : 0)) * kBQ + w * 32 + n;
      float* po = a.part_o + row * kHeadDim;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(po + db * 32 + g * 8 + hh * 4) =
              f32x4{oacc[db][g * 4] * ig, oacc[db][g * 4 + 1] * ig, oacc[db][g * 4 + 2] * ig,
                    oacc[db][g * 4 + 3] * ig};
      if (hh == 0) *reinterpret_cast<float2*>(a.part_ml + row * 2) = make_float2(m_run, l_tot);
    }
    continue;
  }
  const float inv = l_tot > 0.f ? 1.0f / (l_tot * G) : 0.f;
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
}

// ---------------------------------------------------------------------------------------------
// Merge of the split q-tiles (AttnArgs.split): workgroup qg of the grid owns q-tile qg.  It finds
// the split workgroups whose unit ranges cover the q-tile's units [qg*nt, (qg+1)*nt) and
// combines their records per query row: M = max m_p, O = sum 2^(m_p - M) O_p / sum 2^(m_p - M)
// l_p (a record with m_p = -inf has O_p = 0, l_p = 0).  A q-tile inside one workgroup's range was
// written by attn_kernel itself.  Workgroup (qg, g) merges rows 32g .. 32g+31 of q-tile qg: half a
// wave per row and 4 channels (one PRoPE group) per lane, each lane on kCombineRows rows 8 apart
// whose loads are issued together, so one record search serves 32 rows and the loads of a lane's
// rows overlap.
constexpr int kSplitBQ = 256;     // queries per q-tile of the split (8-wave) kernel
constexpr int kMaxSplitWg = 1024;  // split grids have at most this many workgroups
constexpr int kCombineRows = 4;    // rows per lane of attn_combine_kernel
constexpr int kCombineWgs = kSplitBQ / (8 * kCombineRows);  // its workgroups per q-tile

template <typename QT>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  __shared__ int64_t recs[kMaxSplitWg];
  __shared__ int n_rec;
  const int nt = a.nt;
  const int qg = blockIdx.x / kCombineWgs, rg = blockIdx.x % kCombineWgs;
  const int64_t x0 = (int64_t)qg * nt, x1 = x0 + nt - 1;
  auto lo = [&](int i) { return (int64_t)i * a.units / a.n_wg; };
  auto owner = [&](int64_t x) {  // the workgroup whose range holds unit x
    int i = (int)(x * a.n_wg / a.units);
    while (i + 1 < a.n_wg && lo(i + 1) <= x) ++i;
    while (i > 0 && lo(i) > x) --i;
    return i;
  };
  const int i0 = owner(x0), i1 = owner(x1);
  if (i0 == i1) return;  // uniform: one workgroup covered the q-tile and wrote it
  if (threadIdx.x == 0) {  // the records of this q-tile, once
    int m = 0;
    for (int i = i0; i <= i1; ++i)
      if (lo(i) < lo(i + 1)) recs[m++] = 2 * (int64_t)i + (i == i0 && lo(i) < x0 ? 1 : 0);
    n_rec = m;
  }
  __syncthreads();
  const int nr = n_rec;
  const int qt = (qg + a.qt_base) % a.n_qtiles, bh = (qg + a.qt_base) / a.n_qtiles;
  const int h = bh % a.H, b = bh / a.H;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = (lane & 31) * 4;
  const int r0 = rg * (8 * kCombineRows) + 2 * w + (lane >> 5);  // rows r0 + 8 j
  // rows past Lq read records in bounds (every record holds kSplitBQ rows) and store nothing
  float M[kCombineRows];
#pragma unroll
  for (int j = 0; j < kCombineRows; ++j) M[j] = -INFINITY;
  for (int p = 0; p < nr; ++p) {
#pragma unroll
    for (int j = 0; j < kCombineRows; ++j)
      M[j] = fmaxf(M[j], a.part_ml[(recs[p] * kSplitBQ + r0 + 8 * j) * 2]);
  }
  float L[kCombineRows], o[kCombineRows][4];
#pragma unroll
  for (int j = 0; j < kCombineRows; ++j) {
    L[j] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[j][e] = 0.f;
  }
  for (int p = 0; p < nr; ++p) {
#pragma unroll
    for (int j = 0; j < kCombineRows; ++j) {
      const int64_t row = recs[p] * kSplitBQ + r0 + 8 * j;
      const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + row * 2);
      if (ml.x == -INFINITY) continue;
      const float wgt = __builtin_amdgcn_exp2f(ml.x - M[j]);
      const f32x4 v = *reinterpret_cast<const f32x4*>(a.part_o + row * kHeadDim + c);
      L[j] = fmaf(wgt, ml.y, L[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[j][e] = fmaf(wgt, v[e], o[j][e]);
    }
  }
#pragma unroll
  for (int j = 0; j < kCombineRows; ++j) {
    const int qrow = qt * kSplitBQ + r0 + 8 * j;
    if (qrow >= a.Lq) break;  // rows grow with j
    const float inv = L[j] > 0.f ? 1.0f / L[j] : 0.f;
    float x0v = o[j][0] * inv, x1v = o[j][1] * inv, x2v = o[j][2] * inv, x3v = o[j][3] * inv;
    if (a.pq_o) {  // PRoPE: P_q of the query's frame on every group of the output
      const float* po = a.pq_o + ((int64_t)b * a.n_qframes + qrow / a.T) * 16;
      const float y0 = fmaf(po[0], x0v, fmaf(po[1], x1v, fmaf(po[2], x2v, po[3] * x3v)));
      const float y1 = fmaf(po[4], x0v, fmaf(po[5], x1v, fmaf(po[6], x2v, po[7] * x3v)));
      const float y2 = fmaf(po[8], x0v, fmaf(po[9], x1v, fmaf(po[10], x2v, po[11] * x3v)));
      const float y3 = fmaf(po[12], x0v, fmaf(po[13], x1v, fmaf(po[14], x2v, po[15] * x3v)));
      x0v = y0, x1v = y1, x2v = y2, x3v = y3;
    }
    QT* op = static_cast<QT*>(a.o) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qrow * a.o_st;
    store4<QT>(op + c, x0v, x1v, x2v, x3v);
  }
}

}  // namespace skv

using namespace skv;

int skv::cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

// Bytes of the balanced split's records: 2 per workgroup (one per partial segment) of kSplitBQ
// rows, each row 128 O floats plus the running max and sum.
static int64_t split_workspace_bytes(int n_wg) {
  return (int64_t)2 * n_wg * kSplitBQ * (kHeadDim + 2) * (int64_t)sizeof(float);
}

template <int NW>
static void launch(const AttnArgs& a, int q_dtype, int pool_dtype, int rm, hipStream_t s) {
  dim3 grid(a.n_wg), block(NW * 64);
  if (pool_dtype == SKV_F16) {  // plain attention, f16 MFMAs; q f16 or f32 (checked by the caller)
    const bool qh = q_dtype == SKV_F16;
    if constexpr (NW == 8) {
      if (a.split) {
        if (a.packed) {
          if (qh) hipLaunchKernelGGL((attn_kernel<NW, f16, f16, 0, true, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, true), s, a);
          else hipLaunchKernelGGL((attn_kernel<NW, float, f16, 0, true, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, true), s, a);
        } else {
          if (qh) hipLaunchKernelGGL((attn_kernel<NW, f16, f16, 0, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, false), s, a);
          else hipLaunchKernelGGL((attn_kernel<NW, float, f16, 0, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, false), s, a);
        }
        return;
      }
    }
    if (a.packed) {
      if (qh) hipLaunchKernelGGL((attn_kernel<NW, f16, f16, 0, false, true>), grid, block, attn_lds_bytes(NW, 0, 2, false, true), s, a);
      else hipLaunchKernelGGL((attn_kernel<NW, float, f16, 0, false, true>), grid, block, attn_lds_bytes(NW, 0, 2, false, true), s, a);
    } else {
      if (qh) hipLaunchKernelGGL((attn_kernel<NW, f16, f16, 0>), grid, block, attn_lds_bytes(NW, 0, 2, false, false), s, a);
      else hipLaunchKernelGGL((attn_kernel<NW, float, f16, 0>), grid, block, attn_lds_bytes(NW, 0, 2, false, false), s, a);
    }
    return;
  }
  // fp8 pools with RoPE on load: the fp8-MFMA kernel (query temporal pairs rebuilt per key
  // frame) when a q-tile spans at most kFp8TabFrames query frames (frames of >= 64 tokens);
  // shorter frames and fused PRoPE take the bf16 kernel staging decoded tiles (PRoPE's
  // per-key-frame W is unbounded, so the query cannot keep one fp8 scale).  bf16 queries
  // (checked by the caller).
  if (pool_dtype == SKV_FP8_E4M3 && rm == 1 && a.T < kTile) {
    if constexpr (NW == 8) {
      if (a.split) {
        hipLaunchKernelGGL((attn_kernel<NW, bf16, fp8e4, 1, true>), grid, block, attn_lds_bytes(NW, 1, 1, true, false), s, a);
        return;
      }
    }
    hipLaunchKernelGGL((attn_kernel<NW, bf16, fp8e4, 1>), grid, block, attn_lds_bytes(NW, 1, 1, false, false), s, a);
    return;
  }
  if (pool_dtype == SKV_FP8_E4M3 && rm == 1) {
    if constexpr (NW == 8) {
      if (a.split) {
        hipLaunchKernelGGL((attn_fp8_kernel<NW, bf16, true, 1>), grid, block, fp8_lds_bytes(NW, 1), s, a);
        return;
      }
    }
    hipLaunchKernelGGL((attn_fp8_kernel<NW, bf16, false, 1>), grid, block, fp8_lds_bytes(NW, 1), s, a);
    return;
  }
  if (pool_dtype == SKV_FP8_E4M3 && rm == 2) {  // bf16 queries (checked by the caller)
    if constexpr (NW == 8) {
      if (a.split) {
        hipLaunchKernelGGL((attn_kernel<NW, bf16, fp8e4, 2, true>), grid, block, attn_lds_bytes(NW, 2, 1, true, false), s, a);
        return;
      }
    }
    hipLaunchKernelGGL((attn_kernel<NW, bf16, fp8e4, 2>), grid, block, attn_lds_bytes(NW, 2, 1, false, false), s, a);
    return;
  }
  if (pool_dtype == SKV_FP8_E4M3) {
    if constexpr (NW == 8) {
      if (a.split) {
        if (q_dtype == SKV_BF16)
          hipLaunchKernelGGL((attn_fp8_kernel<NW, bf16, true>), grid, block, fp8_lds_bytes(NW), s, a);
        else
          hipLaunchKernelGGL((attn_fp8_kernel<NW, float, true>), grid, block, fp8_lds_bytes(NW), s, a);
        return;
      }
    }
    if (q_dtype == SKV_BF16)
      hipLaunchKernelGGL((attn_fp8_kernel<NW, bf16>), grid, block, fp8_lds_bytes(NW), s, a);
    else
      hipLaunchKernelGGL((attn_fp8_kernel<NW, float>), grid, block, fp8_lds_bytes(NW), s, a);
    return;
  }
  if constexpr (NW == 8) {
    if (a.split) {  // bf16 or fp32 pools, no mask (checked by the caller)
      const bool qb = q_dtype == SKV_BF16;
      if (rm == 2) {
        if (qb) hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 2, true>), grid, block, attn_lds_bytes(NW, 2, 2, true, false), s, a);
        else hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 2, true>), grid, block, attn_lds_bytes(NW, 2, 2, true, false), s, a);
      } else if (rm == 1) {
        if (qb) hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 1, true>), grid, block, attn_lds_bytes(NW, 1, 2, true, false), s, a);
        else hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 1, true>), grid, block, attn_lds_bytes(NW, 1, 2, true, false), s, a);
      } else if (pool_dtype == SKV_BF16 && a.packed) {
        if (qb) hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 0, true, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, true), s, a);
        else hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 0, true, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, true), s, a);
      } else if (pool_dtype == SKV_BF16) {
        if (qb) hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 0, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, false), s, a);
        else hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 0, true>), grid, block, attn_lds_bytes(NW, 0, 2, true, false), s, a);
      } else {
        if (qb) hipLaunchKernelGGL((attn_kernel<NW, bf16, float, 0, true>), grid, block, attn_lds_bytes(NW, 0, 4, true, false), s, a);
        else hipLaunchKernelGGL((attn_kernel<NW, float, float, 0, true>), grid, block, attn_lds_bytes(NW, 0, 4, true, false), s, a);
      }
      return;
    }
  }
  if (rm == 2) {  // bf16 pools, frame_tokens >= 64 (checked by the caller)
    if (q_dtype == SKV_BF16)
      hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 2>), grid, block, attn_lds_bytes(NW, 2, 2, false, false), s, a);
    else
      hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 2>), grid, block, attn_lds_bytes(NW, 2, 2, false, false), s, a);
    return;
  }
  if (rm == 1) {  // bf16 pools only (checked by the caller)
    if (q_dtype == SKV_BF16)
      hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 1>), grid, block, attn_lds_bytes(NW, 1, 2, false, false), s, a);
    else
      hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 1>), grid, block, attn_lds_bytes(NW, 1, 2, false, false), s, a);
    return;
  }
  if (pool_dtype == SKV_BF16 && a.packed) {
    if (q_dtype == SKV_BF16)
      hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 0, false, true>), grid, block, attn_lds_bytes(NW, 0, 2, false, true), s, a);
    else
      hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 0, false, true>), grid, block, attn_lds_bytes(NW, 0, 2, false, true), s, a);
  } else if (q_dtype == SKV_BF16 && pool_dtype == SKV_BF16)
    hipLaunchKernelGGL((attn_kernel<NW, bf16, bf16, 0>), grid, block, attn_lds_bytes(NW, 0, 2, false, false), s, a);
  else if (q_dtype == SKV_BF16 && pool_dtype == SKV_F32)
    hipLaunchKernelGGL((attn_kernel<NW, bf16, float, 0>), grid, block, attn_lds_bytes(NW, 0, 4, false, false), s, a);
  else if (q_dtype == SKV_F32 && pool_dtype == SKV_BF16)
    hipLaunchKernelGGL((attn_kernel<NW, float, bf16, 0>), grid, block, attn_lds_bytes(NW, 0, 2, false, false), s, a);
  else
    hipLaunchKernelGGL((attn_kernel<NW, float, float, 0>), grid, block, attn_lds_bytes(NW, 0, 4, false, false), s, a);
}

static int attention_impl(const void* q, int q_dtype, int64_t q_sb, int64_t q_st,
                          int64_t q_sh, const void* k_pool, const void* v_pool,
                          const float* k_scale, const float* v_scale, int pool_dtype,
                          int n_slots, const int32_t* frame_slots, int n_frames, int batch,
                          int heads, int head_dim, int q_len, int frame_tokens,
                          float softmax_scale, int mask_mode, int64_t q_pos0,
                          int64_t chunk_tokens, void* out, int64_t out_sb, int64_t out_st,
                          int64_t out_sh, const float* rope_hw, int grid_h, int grid_w,
                          const float* rope_t, int n_qframes, const float* pq_t,
                          const float* pq_s, const float* pq_o, skv_stream_t stream,
                          const float* q_inv_rms = nullptr, int64_t q_rms_sb = 0,
                          const float* q_norm_weight = nullptr,
                          const int32_t* frame_lens = nullptr, void* workspace = nullptr,
                          int64_t workspace_bytes = 0, skv_launch_plan* plan = nullptr,
                          const int32_t* seg_rows = nullptr, const int32_t* seg_frames = nullptr,
                          int n_segments = 0) {
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
  if (!(q_dtype == SKV_BF16 || q_dtype == SKV_F32 || q_dtype == SKV_F16)) {
    set_error("skv_attention: q_dtype=%d unsupported", q_dtype);
    return SKV_E_UNSUPPORTED;
  }
  if (!(pool_dtype == SKV_BF16 || pool_dtype == SKV_F32 || pool_dtype == SKV_FP8_E4M3 ||
        pool_dtype == SKV_F16)) {
    set_error("skv_attention: pool_dtype=%d unsupported", pool_dtype);
    return SKV_E_UNSUPPORTED;
  }
  // f16 pools take f16 or f32 queries, f16 queries need f16 pools (the reference casts q to the
  // key/value dtype before its kernel, attention.py:86-87)
  const bool q_ok = pool_dtype == SKV_F16 ? (q_dtype == SKV_F16 || q_dtype == SKV_F32)
                                          : q_dtype != SKV_F16;
  if (!q_ok) {
    set_error("skv_attention: q_dtype=%d with pool_dtype=%d unsupported (f16 pools take f16 or "
              "f32 queries; f16 queries need f16 pools)", q_dtype, pool_dtype);
    return SKV_E_UNSUPPORTED;
  }
  if (pool_dtype == SKV_FP8_E4M3 && (!k_scale || !v_scale)) {
    set_error("skv_attention: fp8 pools need k_scale and v_scale");
    return SKV_E_ARG;
  }
  if (q_sb % 8 || q_st % 8 || q_sh % 8 || out_sb % 4 || out_st % 4 || out_sh % 4) {
    set_error("skv_attention: q strides must be multiples of 8 and out strides of 4 elements");
    return SKV_E_ARG;
  }
  if ((int64_t)n_frames * padded_tokens(frame_tokens) >= ((int64_t)1 << 31)) {
    set_error("skv_attention: key window of %d frames x %d tokens exceeds 2^31", n_frames,
              frame_tokens);
    return SKV_E_ARG;
  }
  if ((q_inv_rms == nullptr) != (q_norm_weight == nullptr)) {
    set_error("skv_attention_ex: Q RMSNorm needs both q_inv_rms and q_norm_weight");
    return SKV_E_ARG;
  }
  if (q_inv_rms && q_rms_sb < q_len) {
    set_error("skv_attention_ex: q_rms_stride_b=%lld < q_len=%d", (long long)q_rms_sb, q_len);
    return SKV_E_ARG;
  }
  const bool prope = pq_t != nullptr;
  const bool rope = rope_t != nullptr || prope;
  if (prope && (!pq_s || !pq_o)) {
    set_error("skv_attention_prope: need q_xform_t, q_xform_s and out_xform");
    return SKV_E_ARG;
  }
  if (prope && (int64_t)batch * n_frames * n_qframes * kWPair >= ((int64_t)1 << 31)) {
    set_error("skv_attention_prope: q_xform_t exceeds 2^31 bytes");
    return SKV_E_ARG;
  }
  if (rope && pool_dtype == SKV_FP8_E4M3 &&
      (int64_t)n_qframes * n_frames * 8 * kRopeT >= ((int64_t)1 << 31)) {
    set_error("skv_attention_rope: rope_t exceeds 2^31 bytes");
    return SKV_E_ARG;
  }
  if (prope && frame_tokens < kTile) {
    set_error("skv_attention_prope: frame_tokens=%d < %d unsupported", frame_tokens, kTile);
    return SKV_E_UNSUPPORTED;
  }
  if (rope) {
    // fp8 pools: the bf16 kernel decodes each staged tile with its frame's scale
    if (!(pool_dtype == SKV_BF16 || (pool_dtype == SKV_FP8_E4M3 && q_dtype == SKV_BF16))) {
      set_error("skv_attention_rope: bf16 pools, or fp8 pools with bf16 queries, are supported");
      return SKV_E_UNSUPPORTED;
    }
    if (!rope_hw || grid_h <= 0 || grid_w <= 0 || (int64_t)grid_h * grid_w != frame_tokens ||
        n_qframes <= 0 || (int64_t)n_qframes * frame_tokens != q_len) {
      set_error("skv_attention_rope: need rope_hw, grid_h * grid_w == frame_tokens (%d x %d vs "
                "%d) and q_len == n_qframes * frame_tokens (%d vs %d x %d)", grid_h, grid_w,
                frame_tokens, q_len, n_qframes, frame_tokens);
      return SKV_E_ARG;
    }
  }
  if (workspace_bytes < 0 || (workspace == nullptr && workspace_bytes != 0)) {
    set_error("skv_attention_ex: workspace_bytes=%lld without a workspace pointer",
              (long long)workspace_bytes);
    return SKV_E_ARG;
  }
  // segments: consecutive query ranges, each over its own consecutive run of the frame list
  int64_t seg_qtiles = 0;
  int seg_max_frames = 0;
  if (n_segments != 0) {
    if (n_segments < 0 || n_segments > SKV_MAX_SEGMENTS || !seg_rows || !seg_frames) {
      set_error("skv_attention_ex: n_segments=%d needs seg_rows and seg_frames and at most %d "
                "segments", n_segments, SKV_MAX_SEGMENTS);
      return SKV_E_ARG;
    }
    if (pool_dtype != SKV_BF16 || q_dtype == SKV_F16 || rope || mask_mode != SKV_MASK_NONE) {
      set_error("skv_attention_ex: segments need bf16 pools, bf16 or f32 queries, mask NONE and "
                "no RoPE / PRoPE");
      return SKV_E_UNSUPPORTED;
    }
    int64_t rows = 0, frames = 0;
    for (int sgi = 0; sgi < n_segments; ++sgi) {
      if (seg_rows[sgi] < 1 || seg_frames[sgi] < 1) {
        set_error("skv_attention_ex: segment %d has %d rows and %d frames (both must be >= 1)",
                  sgi, seg_rows[sgi], seg_frames[sgi]);
        return SKV_E_ARG;
      }
      rows += seg_rows[sgi];
      frames += seg_frames[sgi];
      seg_qtiles += (seg_rows[sgi] + 255) / 256;
      seg_max_frames = seg_frames[sgi] > seg_max_frames ? seg_frames[sgi] : seg_max_frames;
    }
    if (rows != q_len || frames != n_frames) {
      set_error("skv_attention_ex: segments cover %lld rows and %lld frames, expected q_len=%d and "
                "n_frames=%d", (long long)rows, (long long)frames, q_len, n_frames);
      return SKV_E_ARG;
    }
  }
  if (q_len == 0) {
    if (plan) *plan = skv_launch_plan{0, 0, 0, 0, 0, 0};
    return SKV_OK;
  }
  AttnArgs a;
  a.rope_hw = rope_hw;
  a.rope_t = rope_t;
  a.pq_t = pq_t;
  a.pq_s = pq_s;
  a.pq_o = pq_o;
  a.q_rms = q_inv_rms;
  a.q_rms_sb = q_rms_sb;
  a.q_w = q_norm_weight;
  a.gh = grid_h;
  a.gw = grid_w;
  a.n_qframes = n_qframes;
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
  // Packed key tiles: with whole frames whose token count is a multiple of 8 but not of 64, the
  // bf16 / f16 kernel runs 64-key tiles across frame boundaries instead of padding each frame to
  // a whole tile (C2: 512 tiles for 21 x 1560 keys instead of 525); V^T's 8-token groups stay
  // inside one frame.  RoPE instances and fp8 / fp32 pools keep frame-aligned tiles (per-frame
  // query rotations and scales; register staging).
  // The packed kernel addresses each pool through one buffer descriptor with 32-bit offsets,
  // so the pool must be smaller than 4 GB.
  {
    bool whole = true;
    for (int j = 0; frame_lens && j < n_frames; ++j) whole &= frame_lens[j] == frame_tokens;
    const int64_t pool_bytes = (int64_t)n_slots * batch * heads * a.Tp * kHeadDim * 2;
    a.packed = (pool_dtype == SKV_BF16 || pool_dtype == SKV_F16) && !rope && whole &&
               frame_tokens >= kTile && frame_tokens % 8 == 0 && frame_tokens % kTile != 0 &&
               pool_bytes < ((int64_t)1 << 32) - 1;
    a.pool_bytes = a.packed ? (uint32_t)pool_bytes : 0u;
  }
  a.nt = a.packed ? (int)(((int64_t)n_frames * frame_tokens + kTile - 1) / kTile)
                  : n_frames * a.ntiles_f;
  // Workgroup shape: 8 waves (256 queries, 1 workgroup per CU) stages half the K/V bytes per
  // query of 4 waves (128 queries, 2 per CU) and measured ~4% faster per FLOP, but a grid that
  // barely spills into a second round of CUs leaves most of the chip idle; pick the shape with
  // the better CU fill (ties and near-ties go to 8 waves).
  const int n_cu = cu_count();
  auto fill = [&](int bq, int per_cu) {
    const int64_t wg = (int64_t)((q_len + bq - 1) / bq) * heads * batch;
    const int64_t slots = (int64_t)n_cu * per_cu;
    return (double)wg / (double)(((wg + slots - 1) / slots) * slots);
  };
  int nw = fill(256, 1) * 1.04 >= fill(128, 2) ? 8 : 4;
  a.n_qtiles = (q_len + nw * 32 - 1) / (nw * 32);
  a.n_seg = n_segments;
  if (n_segments > 0) {  // 8-wave groups; each segment's q-tiles start at its first row
    nw = 8;
    a.n_qtiles = (int)seg_qtiles;
    for (int sgi = 0; sgi < n_segments; ++sgi) {
      a.seg_rows[sgi] = seg_rows[sgi];
      a.seg_nf[sgi] = seg_frames[sgi];
    }
    // key tiles of the longest segment's list (reported by the plan)
    a.nt = a.packed ? (int)(((int64_t)seg_max_frames * frame_tokens + kTile - 1) / kTile)
                    : seg_max_frames * a.ntiles_f;
  }
  a.n_wg = a.n_qtiles * heads * batch;
  // Balanced key split: when the grid leaves many CUs idle (few q-tiles, e.g. one frame of
  // queries), one 8-wave workgroup per CU takes an equal share of all (q-tile, key tile) units;
  // split q-tiles are merged by attn_combine_kernel.  A tile costs more the more CUs are busy
  // (measured on MI355X with 525 tiles per workgroup: 128, 224 and 256 busy CUs take 0.81, 0.92
  // and 1.0 of the full-chip time), modelled as t(busy) ~ 1 + 0.62 * busy / n_cu; the split
  // runs all CUs, plus about three tiles of segment set-up and merge.  Near-full grids (e.g.
  // 228 q-tiles on 256 CUs) gain too little to pay for the merge and stay unsplit.  A pair of
  // 4-wave workgroups costs 1.10 of one 8-wave workgroup per tile (fitted to the C3 shape,
  // H24 x 18480 keys, B 1 and 2), so 4-wave grids split at a smaller margin: the split also
  // moves them onto the 8-wave kernel (C3: 0.598 -> 0.571 ms, B 2: 1.246 -> 1.154 ms).
  a.split = 0;
  a.units = 0;
  a.qt_base = 0;
  a.part_o = a.part_ml = nullptr;
  int64_t split_bytes = 0;
  int split_mode = 0;  // 1: every q-tile shares the CUs; 2: only the last round's q-tiles do
  const int nt = a.nt;
  const int64_t qt8 = (int64_t)((q_len + kSplitBQ - 1) / kSplitBQ) * heads * batch;
  const int64_t units8 = qt8 * nt;
  if (mask_mode == SKV_MASK_NONE && n_segments == 0 && nt >= 8 && units8 >= 4 * n_cu &&
      n_cu <= kMaxSplitWg) {
    auto t_tile = [&](int64_t busy) { return 1.0 + 0.62 * (double)busy / n_cu; };
    auto t_grid = [&](int64_t wg, int per_cu, double per_tile) {  // rounds of nt tiles
      const int64_t slots = (int64_t)n_cu * per_cu, full = wg / slots, last = wg - full * slots;
      return per_tile * nt * (full * t_tile(n_cu) + (last ? t_tile((last + per_cu - 1) / per_cu) : 0.0));
    };
    const double t_plain = nw == 8 ? t_grid(a.n_wg, 1, 1.0) : t_grid(a.n_wg, 2, 1.10);
    const double t_split = ((double)units8 / n_cu + 3.0) * t_tile(n_cu);
    if (t_split < (nw == 8 ? 0.85 : 0.97) * t_plain) {
      split_bytes = split_workspace_bytes(n_cu);
      split_mode = 1;
    } else if (nw == 8 && a.n_wg > n_cu && a.n_wg % n_cu != 0) {
      // tail split: the full rounds run unsplit, the q-tiles of the last, partly filled round
      // share all CUs (C5: 912 q-tiles = 3 rounds + 144; the 4th round would run at 56% fill)
      const int64_t full = a.n_wg / n_cu, last = a.n_wg - full * n_cu;
      const double t_tail = full * nt * t_tile(n_cu) + ((double)last * nt / n_cu + 3.0) * t_tile(n_cu);
      if (t_tail < 0.97 * t_plain) {
        split_bytes = split_workspace_bytes(n_cu);
        split_mode = 2;
      }
    }
  }
  // The split needs the caller's workspace (2 records of kSplitBQ rows x (O, max, sum) per
  // workgroup); without one the launch stays unsplit.  The library never allocates.
  if (split_bytes > 0 && workspace != nullptr) {
    if (workspace_bytes < split_bytes) {
      set_error("skv_attention_ex: workspace of %lld bytes is smaller than the %lld this launch "
                "needs (skv_attention_plan)", (long long)workspace_bytes, (long long)split_bytes);
      return SKV_E_ARG;
    }
    if (reinterpret_cast<uintptr_t>(workspace) % 16) {
      set_error("skv_attention_ex: workspace must be 16-byte aligned");
      return SKV_E_ARG;
    }
    if (split_mode == 1) {
      nw = 8;
      a.split = 1;
      a.n_qtiles = (int)(qt8 / ((int64_t)heads * batch));
      a.n_wg = n_cu;
      a.units = units8;
    } else {
      a.split = 2;  // launched below as an unsplit grid of the full rounds, then the tail
    }
  }
  a.slot_stride = (int64_t)batch * heads * a.Tp * kHeadDim;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.mask_mode = mask_mode;
  a.q_pos0 = q_pos0;
  a.chunk = chunk_tokens > 0 ? chunk_tokens : 1;
  a.n_keys = (int64_t)n_frames * frame_tokens;
  if (frame_lens && frame_tokens > 65535) {
    set_error("skv_attention_ex: frame_lens need frame_tokens <= 65535");
    return SKV_E_UNSUPPORTED;
  }
  bool ragged = false;
  for (int j = 0; j < n_frames; ++j) {
    if (frame_slots[j] < 0 || frame_slots[j] >= n_slots) {
      set_error("skv_attention: frame_slots[%d]=%d outside [0, %d)", j, frame_slots[j], n_slots);
      return SKV_E_ARG;
    }
    a.slots[j] = frame_slots[j];
    const int len = frame_lens ? frame_lens[j] : frame_tokens;
    if (len < 1 || len > frame_tokens) {
      set_error("skv_attention_ex: frame_lens[%d]=%d outside [1, %d]", j, len, frame_tokens);
      return SKV_E_ARG;
    }
    a.flen[j] = (int32_t)len;
    ragged |= len != frame_tokens;
  }
  if (ragged && mask_mode == SKV_MASK_CHUNK_CAUSAL) {
    set_error("skv_attention_ex: the chunk-causal mask needs whole frames (no frame_lens)");
    return SKV_E_UNSUPPORTED;
  }
  const int64_t full_wg = a.split == 2 ? (int64_t)(a.n_wg / n_cu) * n_cu : 0;
  if (plan) {
    *plan = skv_launch_plan{nw, a.split, a.split == 2 ? (int)full_wg + n_cu : a.n_wg,
                            a.n_qtiles * heads * batch, split_bytes, a.nt};
    return SKV_OK;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rm = prope ? 2 : rope ? 1 : 0;
  auto combine = [&](const AttnArgs& c, int n_q) {
    if (q_dtype == SKV_BF16)
      hipLaunchKernelGGL((attn_combine_kernel<bf16>), dim3(n_q * kCombineWgs), dim3(256), 0, s, c);
    else if (q_dtype == SKV_F16)
      hipLaunchKernelGGL((attn_combine_kernel<f16>), dim3(n_q * kCombineWgs), dim3(256), 0, s, c);
    else
      hipLaunchKernelGGL((attn_combine_kernel<float>), dim3(n_q * kCombineWgs), dim3(256), 0, s, c);
  };
  if (a.split) {
    // 2 records per split workgroup (n_cu of them): O rows first, then (max, sum) pairs
    const size_t rec_rows = (size_t)2 * n_cu * kSplitBQ;
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = a.part_o + rec_rows * kHeadDim;
  }
  if (a.split == 2) {
    // the full rounds unsplit, then the last round's q-tiles [full_wg, n_wg) over every CU
    const int n_tail = a.n_wg - (int)full_wg;
    AttnArgs m = a;
    m.split = 0;
    m.n_wg = (int)full_wg;
    launch<8>(m, q_dtype, pool_dtype, rm, s);
    AttnArgs t = a;
    t.split = 1;
    t.n_wg = n_cu;
    t.units = (int64_t)n_tail * nt;
    t.qt_base = (int)full_wg;
    launch<8>(t, q_dtype, pool_dtype, rm, s);
    combine(t, n_tail);
  } else if (a.n_seg > 0) {
    dim3 grid(a.n_wg), block(512);
    const size_t lds = attn_lds_bytes(8, 0, 2, false, a.packed);
    if (a.packed) {
      if (q_dtype == SKV_BF16) hipLaunchKernelGGL((attn_kernel<8, bf16, bf16, 0, false, true, true>), grid, block, lds, s, a);
      else hipLaunchKernelGGL((attn_kernel<8, float, bf16, 0, false, true, true>), grid, block, lds, s, a);
    } else {
      if (q_dtype == SKV_BF16) hipLaunchKernelGGL((attn_kernel<8, bf16, bf16, 0, false, false, true>), grid, block, lds, s, a);
      else hipLaunchKernelGGL((attn_kernel<8, float, bf16, 0, false, false, true>), grid, block, lds, s, a);
    }
  } else {
    if (nw == 8)
      launch<8>(a, q_dtype, pool_dtype, rm, s);
    else
      launch<4>(a, q_dtype, pool_dtype, rm, s);
    if (a.split) combine(a, a.n_qtiles * heads * batch);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("skv_attention: launch failed: %s", hipGetErrorString(e));
    return SKV_E_LAUNCH;
  }
  return SKV_OK;
}

extern "C" int skv_attention(const void* q, int q_dtype, int64_t q_sb, int64_t q_st,
                             int64_t q_sh, const void* k_pool, const void* v_pool,
                             const float* k_scale, const float* v_scale, int pool_dtype,
                             int n_slots, const int32_t* frame_slots, int n_frames, int batch,
                             int heads, int head_dim, int q_len, int frame_tokens,
                             float softmax_scale, int mask_mode, int64_t q_pos0,
                             int64_t chunk_tokens, void* out, int64_t out_sb, int64_t out_st,
                             int64_t out_sh, skv_stream_t stream) {
  clear_error();
  return attention_impl(q, q_dtype, q_sb, q_st, q_sh, k_pool, v_pool, k_scale, v_scale,
                        pool_dtype, n_slots, frame_slots, n_frames, batch, heads, head_dim, q_len,
                        frame_tokens, softmax_scale, mask_mode, q_pos0, chunk_tokens, out, out_sb,
                        out_st, out_sh, nullptr, 0, 0, nullptr, 0, nullptr, nullptr, nullptr,
                        stream);
}

extern "C" int skv_attention_rope(const void* q, int q_dtype, int64_t q_sb, int64_t q_st,
                                  int64_t q_sh, const void* kr_pool, const void* v_pool,
                                  int pool_dtype, int n_slots, const int32_t* frame_slots,
                                  int n_frames, int batch, int heads, int head_dim, int q_len,
                                  int frame_tokens, float softmax_scale, int mask_mode,
                                  int64_t q_pos0, int64_t chunk_tokens, void* out,
                                  int64_t out_sb, int64_t out_st, int64_t out_sh,
                                  const float* rope_hw, int grid_h, int grid_w,
                                  const float* rope_t, int n_qframes, skv_stream_t stream) {
  clear_error();
  if (!rope_t) {
    set_error("skv_attention_rope: null rope_t");
    return SKV_E_ARG;
  }
  return attention_impl(q, q_dtype, q_sb, q_st, q_sh, kr_pool, v_pool, nullptr, nullptr,
                        pool_dtype, n_slots, frame_slots, n_frames, batch, heads, head_dim, q_len,
                        frame_tokens, softmax_scale, mask_mode, q_pos0, chunk_tokens, out, out_sb,
                        out_st, out_sh, rope_hw, grid_h, grid_w, rope_t, n_qframes, nullptr,
                        nullptr, nullptr, stream);
}

extern "C" int skv_attention_prope(const void* q, int q_dtype, int64_t q_sb, int64_t q_st,
                                   int64_t q_sh, const void* kx_pool, const void* vx_pool,
                                   int pool_dtype, int n_slots, const int32_t* frame_slots,
                                   int n_frames, int batch, int heads, int head_dim, int q_len,
                                   int frame_tokens, float softmax_scale, int mask_mode,
                                   int64_t q_pos0, int64_t chunk_tokens, void* out,
                                   int64_t out_sb, int64_t out_st, int64_t out_sh,
                                   const float* rope_hw, int grid_h, int grid_w,
                                   const float* q_xform_t, const float* q_xform_s,
                                   const float* out_xform, int n_qframes, skv_stream_t stream) {
  clear_error();
  if (!q_xform_t) {
    set_error("skv_attention_prope: null q_xform_t");
    return SKV_E_ARG;
  }
  return attention_impl(q, q_dtype, q_sb, q_st, q_sh, kx_pool, vx_pool, nullptr, nullptr,
                        pool_dtype, n_slots, frame_slots, n_frames, batch, heads, head_dim, q_len,
                        frame_tokens, softmax_scale, mask_mode, q_pos0, chunk_tokens, out, out_sb,
                        out_st, out_sh, rope_hw, grid_h, grid_w, nullptr, n_qframes, q_xform_t,
                        q_xform_s, out_xform, stream);
}

static int attention_desc(const skv_attention_desc* d, skv_stream_t stream,
                          skv_launch_plan* plan) {
  clear_error();
  if (!d) {
    set_error("skv_attention_ex: null descriptor");
    return SKV_E_ARG;
  }
  if (d->rope_t && d->q_xform_t) {
    set_error("skv_attention_ex: give rope_t (RoPE) or q_xform_t (RoPE + PRoPE), not both");
    return SKV_E_ARG;
  }
  return attention_impl(d->q, d->q_dtype, d->q_sb, d->q_st, d->q_sh, d->k_pool, d->v_pool,
                        d->k_scale, d->v_scale, d->pool_dtype, d->n_slots, d->frame_slots,
                        d->n_frames, d->batch, d->heads, d->head_dim, d->q_len, d->frame_tokens,
                        d->softmax_scale, d->mask_mode, d->q_pos0, d->chunk_tokens, d->out,
                        d->out_sb, d->out_st, d->out_sh, d->rope_hw, d->grid_h, d->grid_w,
                        d->rope_t, d->n_qframes, d->q_xform_t, d->q_xform_s, d->out_xform, stream,
                        d->q_inv_rms, d->q_rms_stride_b, d->q_norm_weight, d->frame_lens,
                        d->workspace, d->workspace_bytes, plan, d->seg_rows, d->seg_frames,
                        d->n_segments);
}

extern "C" int skv_attention_ex(const skv_attention_desc* d, skv_stream_t stream) {
  return attention_desc(d, stream, nullptr);
}

int skv::attention_with_workspace(const skv_attention_desc* d, void* ws, int64_t ws_bytes,
                                  skv_stream_t stream, skv_launch_plan* plan) {
  if (!d) return attention_desc(d, stream, plan);
  skv_attention_desc local = *d;
  local.workspace = ws;
  local.workspace_bytes = ws ? ws_bytes : 0;
  return attention_desc(&local, stream, plan);
}

extern "C" int skv_attention_plan(const skv_attention_desc* d, skv_launch_plan* plan) {
  if (!plan) {
    clear_error();
    set_error("skv_attention_plan: null plan");
    return SKV_E_ARG;
  }
  return attention_desc(d, nullptr, plan);
}
