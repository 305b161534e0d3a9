// attention.hip -- single-token decode attention over an fp16 KV cache
// (FlashDecoding; reference kernels/attention_decode.cu, ADR 0013), and the
// bridge kernels that connect the fp32 linear path to it (reference
// kernels/attention_bridge.cu): fp32 <-> fp16 casts and the KV-cache append.
//
// Layouts (reference include/engine/kernels.hpp:160-194): q / out [n_heads, D]
// fp16; K / V head-major, key j of KV head h at h * kv_head_stride + j * D;
// query head h reads KV head h / (n_heads / n_kv_heads).
//
// Work mapping on gfx950: one 256-thread workgroup per (group of G query heads
// sharing a KV head, KV split). A lane owns 8 consecutive dims (one 16-byte
// load of K and of V), so D / 8 lanes cover a key and one wave load reads 64 /
// (D / 8) keys (4 at D = 128, 8 at D = 64) as 1 KiB contiguous. Each K / V
// byte is read once for all G heads of the group. Each lane keeps an online
// softmax state (m, l, o[8]) per head in the log2 domain; U key steps are
// processed as a chunk (scores first, one rescale per chunk). Key-lane dot
// products are summed with DPP; states merge exactly -- weights 2^(m_i - m)
// -- across the key lanes of a wave by shuffles, across the 4 waves through
// LDS, and across splits in a merge kernel, always in a fixed order. Splits
// write fp32 (o, m, l) partials to the stream's scratch arena (reused in
// stream order: no allocation or event per call). GQA groups on aligned
// caches (D = 64 or 128) take flash_decode_gqa_wave_kernel instead: the matrix
// cores, K / V loaded straight into MFMA operand registers, 1 to 8 waves per
// split.
#include "gemv_kernels.hpp"
#include "launch.hpp"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <string>
#include <type_traits>

namespace eng {
namespace {

using H8 = gemv::RawVec<_Float16, 8>::type;
using H2 = gemv::RawVec<_Float16, 2>::type;
constexpr int kThreads = 256;
constexpr float kNegInf = -__builtin_huge_valf();

template <bool VEC>
__device__ __forceinline__ H8 load_h8(const _Float16* p) {
  if constexpr (VEC) {
    return __builtin_nontemporal_load(reinterpret_cast<const H8*>(p));
  } else {
    H8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = p[e];
    return r;
  }
}

// Scores and softmax states are kept in the log2 domain (scores scaled by
// scale * log2(e)), so every weight is one hardware exp2: 2^(a - b), 0 for an
// empty state (a == -inf). The output o / l is the same ratio.
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float merge_weight(float a, float b) {
  return a > kNegInf ? __builtin_amdgcn_exp2f(a - b) : 0.0f;
}

// Sum over the LPK (8 or 16) consecutive lanes that hold one key, left in
// every one of them: DPP quad_perm xor-1 and xor-2, then row_half_mirror
// (lane i <- 7 - i within 8 lanes) and, for 16 lanes, row_mirror (i <- 15 - i).
using gemv::dpp_add;
template <int LPK>
__device__ __forceinline__ float sum_key_lanes(float x) {
  static_assert(LPK == 8 || LPK == 16, "8 or 16 lanes per key");
  x = dpp_add<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x = dpp_add<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x = dpp_add<0x141>(x);  // row_half_mirror
  if constexpr (LPK == 16) x = dpp_add<0x140>(x);  // row_mirror
  return x;
}

template <int D, int G, int U, bool VEC, bool PARTIAL>
__global__ __launch_bounds__(kThreads) void flash_decode_split_kernel(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k,
    const _Float16* __restrict__ v, _Float16* __restrict__ out, float* __restrict__ part_o,
    float* __restrict__ part_ml, long long kv_len, long long group_size,
    long long kv_head_stride, float scale, int nsplit) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  constexpr int LPK = D / 8;       // lanes per key
  constexpr int KPW = 64 / LPK;    // keys per wave load
  constexpr int STEP = 4 * KPW;    // keys per workgroup load
  __shared__ float s_m[4][G];
  __shared__ float s_l[4][G];
  __shared__ float s_o[4][G][D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = lane / LPK;
  const int d0 = (lane % LPK) * 8;
  const long long h0 = static_cast<long long>(blockIdx.x) * G;
  const long long kvh = h0 / group_size;
  const int split = static_cast<int>(blockIdx.y);
  const long long j0 = kv_len * split / nsplit;
  const long long j1 = kv_len * (split + 1) / nsplit;
  const float scale2 = scale * kLog2e;

  float qf[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[g][e] = static_cast<float>(q[(h0 + g) * D + d0 + e]);
  }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegInf;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  const _Float16* kh = k + kvh * kv_head_stride + d0;
  const _Float16* vh = v + kvh * kv_head_stride + d0;
  // The loop bound depends on the wave only, so every lane runs the shuffles.
  for (long long jb = j0 + static_cast<long long>(wave) * KPW; jb < j1;
       jb += static_cast<long long>(STEP) * U) {
    H8 kr[U], vr[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long j = jb + static_cast<long long>(u) * STEP + sub;
      ok[u] = j < j1;
      kr[u] = ok[u] ? load_h8<VEC>(kh + j * D) : H8{};
      vr[u] = ok[u] ? load_h8<VEC>(vh + j * D) : H8{};
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[U];
      float cm = kNegInf;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) part = fmaf(qf[g][e], static_cast<float>(kr[u][e]), part);
        part = sum_key_lanes<LPK>(part);
        s[u] = ok[u] ? part * scale2 : kNegInf;
        cm = fmaxf(cm, s[u]);
      }
      const float mn = fmaxf(m[g], cm);
      if (mn > kNegInf) {
        const float alpha = merge_weight(m[g], mn);
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float p = merge_weight(s[u], mn);
          l[g] += p;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] = fmaf(p, static_cast<float>(vr[u][e]), o[g][e]);
        }
        m[g] = mn;
      }
    }
  }

  // Merge the key lanes of the wave (lanes with the same dims, other keys).
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = __shfl_xor(m[g], off);
      const float lo = __shfl_xor(l[g], off);
      const float mn = fmaxf(m[g], mo);
      const float sa = merge_weight(m[g], mn);
      const float sb = merge_weight(mo, mn);
      l[g] = l[g] * sa + lo * sb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float oo = __shfl_xor(o[g][e], off);
        o[g][e] = o[g][e] * sa + oo * sb;
      }
      m[g] = mn;
    }
  }
  if (sub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[wave][g][d0 + e] = o[g][e];
      if (lane == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  for (int idx = tid; idx < G * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    const float mb = fmaxf(fmaxf(s_m[0][g], s_m[1][g]), fmaxf(s_m[2][g], s_m[3][g]));
    float lb = 0.0f, ob = 0.0f;
    if (mb > kNegInf) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float wt = merge_weight(s_m[w][g], mb);
        lb = fmaf(s_l[w][g], wt, lb);
        ob = fmaf(s_o[w][g][d], wt, ob);
      }
    }
    const long long h = h0 + g;
    if constexpr (PARTIAL) {
      const long long slot = h * nsplit + split;
      part_o[slot * D + d] = ob;
      if (d == 0) {
        part_ml[2 * slot] = mb;
        part_ml[2 * slot + 1] = lb;
      }
    } else {
      out[h * D + d] = static_cast<_Float16>(lb > 0.0f ? ob / lb : 0.0f);
    }
  }
}

// GQA decode with K / V tiles staged in LDS: one 256-thread workgroup per (KV
// head's group of G query heads, split). All threads copy a tile of T = 4096
// / D keys of K and V (16 KB) from HBM into LDS, double-buffered: the copy of
// tile t + 1 is in flight while tile t is computed, one barrier per tile. Wave
// w owns HPW = G / 4 query heads (G = 8: 2, G = 4: 1) or, for G = 2, one head
// and every other half-tile (WPH = 2 waves per head); its lanes read K / V
// rows from LDS (16 bytes per lane, a wave read is 1 KiB contiguous) and keep
// the online softmax state of their heads only, so K / V bytes leave HBM once
// per group while the registers hold G / 4 heads, not G.
template <int D, int G, bool VEC, bool PARTIAL>
__global__ __launch_bounds__(kThreads) void flash_decode_gqa_lds_kernel(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k,
    const _Float16* __restrict__ v, _Float16* __restrict__ out, float* __restrict__ part_o,
    float* __restrict__ part_ml, long long kv_len, long long group_size,
    long long kv_head_stride, float scale, int nsplit) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(G == 2 || G == 4 || G == 8, "GQA group of 2, 4 or 8 heads");
  constexpr int LPK = D / 8;                 // lanes per key
  constexpr int KPW = 64 / LPK;              // keys per wave read
  constexpr int T = 4096 / D;                // keys per tile
  constexpr int HPW = G >= 4 ? G / 4 : 1;    // heads per wave
  constexpr int WPH = 4 / (G / HPW);         // waves per head
  constexpr int KEYS = T / WPH;              // keys of a tile per wave
  constexpr int U = KEYS / KPW;              // wave reads per tile
  constexpr int CHUNKS = 2 * T * LPK;        // 16-byte chunks of a K + V tile
  constexpr int CPT = CHUNKS / kThreads;     // chunks per thread
  static_assert(CHUNKS % kThreads == 0 && U >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) _Float16 tile[2][2][T][D];
  __shared__ float s_m[4][HPW];
  __shared__ float s_l[4][HPW];
  __shared__ float s_o[4][HPW][D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = lane / LPK;
  const int d0 = (lane % LPK) * 8;
  const int hslot = wave % (G / HPW);        // which HPW heads of the group
  const int kslice = wave / (G / HPW);       // which key slice of each tile
  const long long hg0 = static_cast<long long>(blockIdx.x) * G;
  const long long kvh = hg0 / group_size;
  const int split = static_cast<int>(blockIdx.y);
  const long long j0 = kv_len * split / nsplit;
  const long long j1 = kv_len * (split + 1) / nsplit;
  const long long ntiles = (j1 - j0 + T - 1) / T;
  const float scale2 = scale * kLog2e;

  float qf[HPW][8];
#pragma unroll
  for (int g = 0; g < HPW; ++g) {
    const long long h = hg0 + hslot * HPW + g;
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[g][e] = static_cast<float>(q[h * D + d0 + e]);
  }
  float m[HPW], l[HPW], o[HPW][8];
#pragma unroll
  for (int g = 0; g < HPW; ++g) {
    m[g] = kNegInf;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  const _Float16* kb = k + kvh * kv_head_stride;
  const _Float16* vb = v + kvh * kv_head_stride;
  H8 stage[CPT];
  auto fetch = [&](long long t) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kThreads;
      const int sel = c / (T * LPK);
      const int r = c - sel * (T * LPK);
      const int key = r / LPK;
      const int col = r - key * LPK;
      const long long j = j0 + t * T + key;
      const _Float16* src = (sel == 0 ? kb : vb) + j * D + col * 8;
      stage[i] = j < j1 ? load_h8<VEC>(src) : H8{};
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * kThreads;
      const int sel = c / (T * LPK);
      const int r = c - sel * (T * LPK);
      const int key = r / LPK;
      const int col = r - key * LPK;
      *reinterpret_cast<H8*>(&tile[buf][sel][key][col * 8]) = stage[i];
    }
  };

  if (ntiles > 0) {
    fetch(0);
    commit(0);
  }
  __syncthreads();
  for (long long t = 0; t < ntiles; ++t) {
    const int buf = static_cast<int>(t & 1);
    if (t + 1 < ntiles) fetch(t + 1);
    const long long tbase = j0 + t * T;
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
      float s[U];
      float cm = kNegInf;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int key = kslice * KEYS + u * KPW + sub;
        const H8 kr = *reinterpret_cast<const H8*>(&tile[buf][0][key][d0]);
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) part = fmaf(qf[g][e], static_cast<float>(kr[e]), part);
        part = sum_key_lanes<LPK>(part);
        s[u] = tbase + key < j1 ? part * scale2 : kNegInf;
        cm = fmaxf(cm, s[u]);
      }
      const float mn = fmaxf(m[g], cm);
      if (mn > kNegInf) {
        const float alpha = merge_weight(m[g], mn);
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int key = kslice * KEYS + u * KPW + sub;
          const float p = merge_weight(s[u], mn);
          const H8 vr = *reinterpret_cast<const H8*>(&tile[buf][1][key][d0]);
          l[g] += p;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] = fmaf(p, static_cast<float>(vr[e]), o[g][e]);
        }
        m[g] = mn;
      }
    }
    if (t + 1 < ntiles) commit(buf ^ 1);
    __syncthreads();
  }

  // Merge the key lanes of the wave.
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
      const float mo = __shfl_xor(m[g], off);
      const float lo = __shfl_xor(l[g], off);
      const float mn = fmaxf(m[g], mo);
      const float sa = merge_weight(m[g], mn);
      const float sb = merge_weight(mo, mn);
      l[g] = l[g] * sa + lo * sb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float oo = __shfl_xor(o[g][e], off);
        o[g][e] = o[g][e] * sa + oo * sb;
      }
      m[g] = mn;
    }
  }
  if (sub == 0) {
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[wave][g][d0 + e] = o[g][e];
      if (lane == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  // Combine the WPH waves of each head (in wave order) and write.
  for (int idx = tid; idx < G * D; idx += kThreads) {
    const int gh = idx / D;                  // head within the group
    const int d = idx - gh * D;
    const int hs = gh / HPW;                 // head slot
    const int g = gh - hs * HPW;
    float mb = kNegInf;
#pragma unroll
    for (int w = 0; w < WPH; ++w) mb = fmaxf(mb, s_m[hs + w * (G / HPW)][g]);
    float lb = 0.0f, ob = 0.0f;
    if (mb > kNegInf) {
#pragma unroll
      for (int w = 0; w < WPH; ++w) {
        const int ww = hs + w * (G / HPW);
        const float wt = merge_weight(s_m[ww][g], mb);
        lb = fmaf(s_l[ww][g], wt, lb);
        ob = fmaf(s_o[ww][g][d], wt, ob);
      }
    }
    const long long h = hg0 + gh;
    if constexpr (PARTIAL) {
      const long long slot = h * nsplit + split;
      part_o[slot * D + d] = ob;
      if (d == 0) {
        part_ml[2 * slot] = mb;
        part_ml[2 * slot + 1] = lb;
      }
    } else {
      out[h * D + d] = static_cast<_Float16>(lb > 0.0f ? ob / lb : 0.0f);
    }
  }
}

// Direct-to-LDS variant for 16-byte aligned caches (any G of 1, 2, 4, 8):
// the same work split and arithmetic as flash_decode_gqa_lds_kernel (G = 1:
// four waves per head, each a quarter of every tile), but the K / V tiles are
// loaded straight into LDS (global_load_lds_dwordx4: lane l writes 16 bytes
// at the wave's LDS base + 16 l) through NST = 4 stages, so three tiles are in
// flight while one is computed and no registers hold staged data. A tile is
// T keys of K and of V, each 8 KiB contiguous in the cache; keys past the
// split's end are loaded from its last key (in bounds, finite) and masked to
// a -inf score. The stages are separate LDS variables and the tile loop is
// unrolled by NST, so every LDS access names its stage statically: the
// compiler then need not make a fragment read wait for the loads in flight
// into the other stages. Each thread issues the same CPT loads per tile, and
// waits with vmcnt = CPT x (tiles issued after the one it needs).
template <int CPT>
__device__ __forceinline__ void wait_tiles_after(int outstanding) {
#if defined(__HIP_DEVICE_COMPILE__)
  if (outstanding >= 2) {
    __builtin_amdgcn_s_waitcnt(vmcnt_le(2 * CPT));
  } else if (outstanding == 1) {
    __builtin_amdgcn_s_waitcnt(vmcnt_le(CPT));
  } else {
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
  }
#endif
}

template <int D, int G, bool PARTIAL>
__global__ __launch_bounds__(kThreads) void flash_decode_gqa_dma_kernel(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k,
    const _Float16* __restrict__ v, _Float16* __restrict__ out, float* __restrict__ part_o,
    float* __restrict__ part_ml, long long kv_len, long long group_size,
    long long kv_head_stride, float scale, int nsplit) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "1, 2, 4 or 8 heads per workgroup");
  constexpr int NST = 4;                     // pipeline stages
  constexpr int LPK = D / 8;                 // lanes per key
  constexpr int KPW = 64 / LPK;              // keys per wave read
  constexpr int T = 4096 / D;                // keys per tile
  constexpr int HPW = G >= 4 ? G / 4 : 1;    // heads per wave
  constexpr int WPH = 4 / (G / HPW);         // waves per head
  constexpr int KEYS = T / WPH;              // keys of a tile per wave
  constexpr int U = KEYS / KPW;              // wave reads per tile
  constexpr int HALF_CHUNKS = T * LPK;       // 16-byte chunks of the K (or V) tile
  constexpr int CPH = HALF_CHUNKS / kThreads;  // loads per thread per K (or V) tile
  constexpr int CPT = 2 * CPH;               // loads per thread per tile
  static_assert(HALF_CHUNKS % kThreads == 0 && U >= 1, "tile shape");
  // Stage s: K tile at S_s[0, T D), V tile at S_s[T D, 2 T D).
  __shared__ __attribute__((aligned(1024))) _Float16 S0[2 * T * D], S1[2 * T * D], S2[2 * T * D],
      S3[2 * T * D];
  __shared__ float s_m[4][HPW];
  __shared__ float s_l[4][HPW];
  __shared__ float s_o[4][HPW][D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = lane / LPK;
  const int d0 = (lane % LPK) * 8;
  const int hslot = wave % (G / HPW);        // which HPW heads of the group
  const int kslice = wave / (G / HPW);       // which key slice of each tile
  const long long hg0 = static_cast<long long>(blockIdx.x) * G;
  const long long kvh = hg0 / group_size;
  const int split = static_cast<int>(blockIdx.y);
  const long long j0 = kv_len * split / nsplit;
  const long long j1 = kv_len * (split + 1) / nsplit;
  const int ntiles = static_cast<int>((j1 - j0 + T - 1) / T);
  const float scale2 = scale * kLog2e;

  // q stays fp16: the scores are v_dot2 (two exact fp16 products added to an
  // fp32 accumulator) of q and K pairs.
  H2 qh[HPW][4];
#pragma unroll
  for (int g = 0; g < HPW; ++g) {
    const long long h = hg0 + hslot * HPW + g;
#pragma unroll
    for (int p = 0; p < 4; ++p) qh[g][p] = H2{q[h * D + d0 + 2 * p], q[h * D + d0 + 2 * p + 1]};
  }
  float m[HPW], l[HPW], o[HPW][8];
#pragma unroll
  for (int g = 0; g < HPW; ++g) {
    m[g] = kNegInf;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  const _Float16* kb = k + kvh * kv_head_stride;
  const _Float16* vb = v + kvh * kv_head_stride;
  // Loads of tile t into one stage: the thread's i-th load of the K (V) tile
  // fills chunk slot (4 i + wave) * 64 + lane, i.e. key slot / LPK, dims
  // (slot % LPK) * 8 .. + 7.
  auto fetch = [&](_Float16* st, int t) __attribute__((always_inline)) {
    _Float16* ks = st;
    _Float16* vs = st + T * D;
#pragma unroll
    for (int i = 0; i < CPH; ++i) {
      const int slot0 = (4 * i + wave) * 64;
      const int slot = slot0 + lane;
      long long j = j0 + static_cast<long long>(t) * T + slot / LPK;
      j = j < j1 ? j : j1 - 1;
      const long long off = j * D + (slot % LPK) * 8;
      dma16(kb + off, ks + 8 * slot0);
      dma16(vb + off, vs + 8 * slot0);
    }
  };
  // One resident tile. Each K row is read once for the wave's HPW heads;
  // each head's state is rescaled once; each V row is read and converted to
  // fp32 once, then accumulated into every head with plain FMAs (a mixed
  // fp16 x fp32 FMA per head would repeat the conversion at a lower rate).
  // An all -inf state stays empty: its weights 2^(s - m) are 0.
  auto compute = [&](const _Float16* st, int t) __attribute__((always_inline)) {
    const _Float16* ks = st;
    const _Float16* vs = st + T * D;
    const long long tbase = j0 + static_cast<long long>(t) * T;
    float sc[HPW][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int key = kslice * KEYS + u * KPW + sub;
      const bool valid = tbase + key < j1;
      const H8 kr = *reinterpret_cast<const H8*>(ks + key * D + d0);
#pragma unroll
      for (int g = 0; g < HPW; ++g) {
        float part = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p)
          part = __builtin_amdgcn_fdot2(qh[g][p], H2{kr[2 * p], kr[2 * p + 1]}, part, false);
        part = sum_key_lanes<LPK>(part);
        sc[g][u] = valid ? part * scale2 : kNegInf;
      }
    }
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
      float cm = sc[g][0];
#pragma unroll
      for (int u = 1; u < U; ++u) cm = fmaxf(cm, sc[g][u]);
      const float mn = fmaxf(m[g], cm);
      const float alpha = merge_weight(m[g], mn);
      l[g] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
      m[g] = mn;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int key = kslice * KEYS + u * KPW + sub;
      const H8 vr = *reinterpret_cast<const H8*>(vs + key * D + d0);
      float vf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vf[e] = static_cast<float>(vr[e]);
        // Materialise the fp32 value once: otherwise the conversion is folded
        // into a mixed-precision FMA for every head.
        asm("" : "+v"(vf[e]));
      }
#pragma unroll
      for (int g = 0; g < HPW; ++g) {
        const float p = merge_weight(sc[g][u], m[g]);
        l[g] += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(p, vf[e], o[g][e]);
      }
    }
  };
  // Step t on stage S: refill the stage step t - 1 used with tile t + NST - 1,
  // compute tile t, then wait for tile t + 1 and meet at the barrier.
  auto step = [&](const _Float16* st, _Float16* next, int t) __attribute__((always_inline)) {
    if (t + NST - 1 < ntiles) fetch(next, t + NST - 1);
    compute(st, t);
    const int last_issued = t + NST - 1 < ntiles - 1 ? t + NST - 1 : ntiles - 1;
    wait_tiles_after<CPT>(last_issued - (t + 1));
    barrier_no_fence();
  };

  // Prologue: tiles 0 .. NST - 2 in flight, tile 0 resident.
  fetch(S0, 0);
  if (1 < ntiles) fetch(S1, 1);
  if (2 < ntiles) fetch(S2, 2);
  {
    const int last_issued = ntiles - 1 < NST - 2 ? ntiles - 1 : NST - 2;
    wait_tiles_after<CPT>(last_issued);
    barrier_no_fence();
  }
  // Steady state (every step refills a stage and leaves two tiles in flight):
  // no branches around the loads or waits, so the compiler's own wait
  // analysis stays exact. Then the last tiles, with the general step.
  auto steady = [&](const _Float16* st, _Float16* next, int t) __attribute__((always_inline)) {
    fetch(next, t + NST - 1);
    compute(st, t);
    wait_tiles_after<CPT>(2);
    barrier_no_fence();
  };
  int t = 0;
  for (; t + 2 * NST - 2 < ntiles; t += NST) {
    steady(S0, S3, t);
    steady(S1, S0, t + 1);
    steady(S2, S1, t + 2);
    steady(S3, S2, t + 3);
  }
  for (; t < ntiles; t += NST) {
    step(S0, S3, t);
    if (t + 1 < ntiles) step(S1, S0, t + 1);
    if (t + 2 < ntiles) step(S2, S1, t + 2);
    if (t + 3 < ntiles) step(S3, S2, t + 3);
  }

  // Merge the key lanes of the wave.
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
      const float mo = __shfl_xor(m[g], off);
      const float lo = __shfl_xor(l[g], off);
      const float mn = fmaxf(m[g], mo);
      const float sa = merge_weight(m[g], mn);
      const float sb = merge_weight(mo, mn);
      l[g] = l[g] * sa + lo * sb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float oo = __shfl_xor(o[g][e], off);
        o[g][e] = o[g][e] * sa + oo * sb;
      }
      m[g] = mn;
    }
  }
  if (sub == 0) {
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[wave][g][d0 + e] = o[g][e];
      if (lane == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  // Combine the WPH waves of each head (in wave order) and write.
  for (int idx = tid; idx < G * D; idx += kThreads) {
    const int gh = idx / D;                  // head within the group
    const int d = idx - gh * D;
    const int hs = gh / HPW;                 // head slot
    const int g = gh - hs * HPW;
    float mb = kNegInf;
#pragma unroll
    for (int w = 0; w < WPH; ++w) mb = fmaxf(mb, s_m[hs + w * (G / HPW)][g]);
    float lb = 0.0f, ob = 0.0f;
    if (mb > kNegInf) {
#pragma unroll
      for (int w = 0; w < WPH; ++w) {
        const int ww = hs + w * (G / HPW);
        const float wt = merge_weight(s_m[ww][g], mb);
        lb = fmaf(s_l[ww][g], wt, lb);
        ob = fmaf(s_o[ww][g][d], wt, ob);
      }
    }
    const long long h = hg0 + gh;
    if constexpr (PARTIAL) {
      const long long slot = h * nsplit + split;
      part_o[slot * D + d] = ob;
      if (d == 0) {
        part_ml[2 * slot] = mb;
        part_ml[2 * slot + 1] = lb;
      }
    } else {
      out[h * D + d] = static_cast<_Float16>(lb > 0.0f ? ob / lb : 0.0f);
    }
  }
}

// GQA decode at D = 64 or 128 for G <= 16 query heads of one KV head: NW
// waves (1, 2, 4 or 8), each owning 32-key blocks (block b of the split goes to wave b % NW) that it
// loads straight into the registers the matrix cores read them from -- no LDS
// staging, no workgroup barrier until the final merge -- with P blocks in
// flight per wave. Per block, on the matrix cores:
//   scores  S^T[32 keys x 16 heads] = K . q^T  (D / 32 v_mfma_f32_16x16x32_f16
//           per 16 keys; fp16 products are exact in fp32, summed in fp32),
//   values  O^T[D dims x 16 heads] += V^T . P^T over the 32 keys, on
//           v_mfma_f32_16x16x32_f16 with the fp32 softmax weights split into two
//           fp16 terms p = hi + lo (hi = fp16(p), lo = fp16(p - hi): 22
//           significant bits, each product exact in fp32), two MFMAs per
//           16-dim block,
// with an online softmax in between, per head in registers, rescaled lazily:
// weights are taken relative to a reference max m that is raised (rescaling o
// and l) only when a block's max exceeds it by more than kLazy (in log2), so
// weights stay <= 2^kLazy before the fixed 2^kWeightShift scale that keeps
// the hi / lo split in fp16's normal range; the final o / l is the same ratio.
// Lane l owns head l % 16 and lane group g = l / 16. MFMA layouts (gfx950):
// A[i][k] is lane i + 16 (k / 8) element k % 8, B[k][j] lane j + 16 (k / 8)
// element k % 8, D[i][j] lane j + 16 (i / 4) element i % 4. Score row
// i = 4 g + e of half-block h is K row 16 h + g + 4 e (A row i loads K row
// 16 h + i / 4 + 4 (i % 4)), so lane group g holds the weights of keys
// {16 h + g + 4 e}; the value step's k index 8 g + e is key
// 16 (e / 4) + g + 4 (e % 4) -- the lane's own weights, in order -- and its A
// operand (V^T, row i = dim VW i + mb of block mb, VW = D / 16) is one load of
// dims VW i .. VW i + VW - 1 per key (8 bytes at D = 64, 16 at D = 128),
// transposed in registers into the D / 16 value blocks, the four lane groups
// reading four consecutive V rows (4 D contiguous bytes per load). A block is
// 2 D bytes per lane: 2 D / 32 16-byte K loads and eight V loads. The waves'
// states merge through LDS in wave order: the output, or an fp32 partial state
// per split.
template <int D, int G, int NW, int P, bool RING, bool PARTIAL>
__global__ __launch_bounds__(64 * NW) void flash_decode_gqa_wave_kernel(
    const _Float16* __restrict__ q, const _Float16* k, const _Float16* v,
    _Float16* __restrict__ out, float* __restrict__ part_o,
    float* __restrict__ part_ml, long long kv_len, long long group_size,
    long long kv_head_stride, float scale, int nsplit) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(G >= 2 && G <= 16, "2 to 16 heads per workgroup");
  static_assert(NW == 1 || NW == 2 || NW == 4 || NW == 8, "1, 2, 4 or 8 waves");
  static_assert(P >= 1 && P <= 4, "1 to 4 blocks in flight per wave");
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  typedef float float4v __attribute__((ext_vector_type(4)));
  constexpr int KS = D / 32;                 // 32-dim steps of a score
  constexpr int VW = D / 16;                 // value blocks = dims per lane per key
  typedef _Float16 halfvw __attribute__((ext_vector_type(VW)));
  constexpr int KB = 32;                     // keys per block
  constexpr int WS = 16 * D + 32;            // floats of one wave's state in LDS
  __shared__ __attribute__((aligned(16))) float s_state[NW > 1 ? NW * WS : 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;
  const long long hg0 = static_cast<long long>(blockIdx.x) * G;
  const long long kvh = hg0 / group_size;
  const int split = static_cast<int>(blockIdx.y);
  const long long j0 = kv_len * split / nsplit;
  const long long j1 = kv_len * (split + 1) / nsplit;
  const int nkeys = static_cast<int>(j1 - j0);
  const int nblocks = (nkeys + KB - 1) / KB;
  const int nb = wave < nblocks ? (nblocks - wave + NW - 1) / NW : 0;  // this wave's blocks
  const float scale2 = scale * kLog2e;

  // q^T as the score B operand (head col, dims 32 ks + 8 grp + j). Columns
  // past G repeat head G - 1 (no load is conditional): they compute its state
  // again, vote as it does in the rescale test, and are never written.
  half8 qb[KS];
  const _Float16* qh = q + (hg0 + min(col, G - 1)) * D + 8 * grp;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int j = 0; j < 8; ++j) qb[ks][j] = qh[32 * ks + j];
  }

  const _Float16* kb = k + kvh * kv_head_stride + j0 * D;
  const _Float16* vb = v + kvh * kv_head_stride + j0 * D;
  struct Block {
    half8 k[2][KS];                          // [half-block][32-dim step]
    halfvw v[8];                             // [k element]
  };
  // Every call issues the same 2 KS + 8 loads, so the compiler's waits count
  // exactly P - 1 blocks in flight behind the one a compute needs. Rows past
  // the split's end load its last key (in bounds; masked below), so a block
  // past this wave's last one is the last key for every lane: one K and one
  // V cache line, never read.
  auto load = [&](Block& b, int t) __attribute__((always_inline)) {
    const int key0 = (wave + NW * t) * KB;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kk = min(key0 + 16 * h + (col >> 2) + 4 * (col & 3), nkeys - 1);
#pragma unroll
      for (int s = 0; s < KS; ++s)
        b.k[h][s] = __builtin_nontemporal_load(
            reinterpret_cast<const half8*>(kb + static_cast<long long>(kk) * D + 32 * s + 8 * grp));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int kk = min(key0 + 16 * (e >> 2) + grp + 4 * (e & 3), nkeys - 1);
      b.v[e] = __builtin_nontemporal_load(
          reinterpret_cast<const halfvw*>(vb + static_cast<long long>(kk) * D + VW * col));
    }
  };

  // max / sum over the four lane groups of a head (lanes l, l ^ 16, l ^ 32,
  // l ^ 48): each swap leaves {x[l], x[l ^ 32]} (then ^ 16) in its two results.
  auto group_max = [](float x) __attribute__((always_inline)) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
  };
  auto group_sum = [](float x) __attribute__((always_inline)) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
  };

  constexpr float kLazy = 8.0f;
  // Weights are 2^(s - m + kWeightShift): at most 2^15 (fp16 holds it), and
  // the fp16 lo term stays normal for weights down to 2^-10 of the max's
  // scale, so those carry 22 significant bits; smaller ones err by at most
  // 2^-32 (unscaled). l and o carry the same factor, so o / l and the merge of
  // split states (all from this kernel) are unchanged.
  constexpr float kWeightShift = 7.0f;
  float m = kNegInf;
  float lsum = 0.0f;
  float4v o[VW];
#pragma unroll
  for (int mb = 0; mb < VW; ++mb) o[mb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](const Block& b, int t) __attribute__((always_inline)) {
    float4v sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b.k[h][0], qb[0], float4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
      for (int ks = 1; ks < KS; ++ks)
        sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b.k[h][ks], qb[ks], sc[h], 0, 0, 0);
    }
    const int kbase = (wave + NW * t) * KB + grp;
    float sv[8];
    float mx = kNegInf;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sv[e] = kbase + 16 * (e >> 2) + 4 * (e & 3) < nkeys ? sc[e >> 2][e & 3] * scale2 : kNegInf;
      mx = fmaxf(mx, sv[e]);
    }
    mx = group_max(mx);
    if (__any(mx > m + kLazy)) {
      const float mn = fmaxf(m, mx);
      const float alpha = merge_weight(m, mn);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int mb = 0; mb < VW; ++mb) o[mb] *= alpha;
    }
    half8 ph, pl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = merge_weight(sv[e], m - kWeightShift);
      lsum += p;
      ph[e] = static_cast<_Float16>(p);
      pl[e] = static_cast<_Float16>(p - static_cast<float>(ph[e]));
    }
    half8 av[VW];
#pragma unroll
    for (int mb = 0; mb < VW; ++mb) {
#pragma unroll
      for (int e = 0; e < 8; ++e) av[mb][e] = b.v[e][mb];
    }
#pragma unroll
    for (int mb = 0; mb < VW; ++mb) o[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[mb], ph, o[mb], 0, 0, 0);
#pragma unroll
    for (int mb = 0; mb < VW; ++mb) o[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[mb], pl, o[mb], 0, 0, 0);
  };

  // Ring of P blocks: block t lives in buf[t % P], every buffer named
  // statically. Without RING the split has at most P blocks per wave (at
  // most 256 P keys): all are loaded at once and the computes run
  // straight-line, each waiting for exactly its own loads. With RING the
  // wave loops over the ring (the compiler's waits at the loop head are
  // coarser there).
  // The loads stay here, in block order: left alone, the compiler sinks a
  // block's loads into the branch that computes it (k and v are not declared
  // __restrict__, so their loads do not move across the asm) and the
  // scheduler interleaves the blocks (the sched_barrier).
  Block buf[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    load(buf[i], i);
    __builtin_amdgcn_sched_barrier(0);
  }
  asm volatile("" ::: "memory");
  if constexpr (!RING) {
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (i < nb) compute(buf[i], i);
  } else {
    for (int t = 0; t < nb; t += P) {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        if (t + i < nb) compute(buf[i], t + i);
        load(buf[i], t + i + P);
      }
    }
  }

  // Lane (col, grp) holds dims VW (4 grp + r) + mb of head col in o[mb][r]:
  // VW consecutive dims per r.
  const float lt = group_sum(lsum);
  if constexpr (NW == 1) {
    // One wave: its state is the workgroup's, written from registers.
    if (col < G) {
      const long long h = hg0 + col;
      if constexpr (PARTIAL) {
        const long long slot = h * nsplit + split;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int c = 0; c < VW; c += 4)
            *reinterpret_cast<float4v*>(part_o + slot * D + VW * (4 * grp + r) + c) =
                float4v{o[c][r], o[c + 1][r], o[c + 2][r], o[c + 3][r]};
        }
        if (grp == 0) {
          part_ml[2 * slot] = m;
          part_ml[2 * slot + 1] = lt;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int mb = 0; mb < VW; ++mb)  // out is only 2-byte aligned
            out[h * D + VW * (4 * grp + r) + mb] = static_cast<_Float16>(lt > 0.0f ? o[mb][r] / lt : 0.0f);
        }
      }
    }
    return;
  }
  // Several waves: each state into LDS (o at [head][dim], then m and l),
  // merged in wave order.
  float* const ws = s_state + wave * WS;
  if (col < G) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int c = 0; c < VW; c += 4)
        *reinterpret_cast<float4v*>(ws + col * D + VW * (4 * grp + r) + c) =
            float4v{o[c][r], o[c + 1][r], o[c + 2][r], o[c + 3][r]};
    }
    if (grp == 0) {
      ws[16 * D + col] = m;
      ws[16 * D + 16 + col] = lt;
    }
  }
  __syncthreads();

  for (int idx = tid; idx < G * D; idx += 64 * NW) {
    const int gh = idx / D;
    const int d = idx - gh * D;
    float mb = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) mb = fmaxf(mb, s_state[w * WS + 16 * D + gh]);
    float lb = 0.0f, ob = 0.0f;
    if (mb > kNegInf) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float wt = merge_weight(s_state[w * WS + 16 * D + gh], mb);
        lb = fmaf(s_state[w * WS + 16 * D + 16 + gh], wt, lb);
        ob = fmaf(s_state[w * WS + gh * D + d], wt, ob);
      }
    }
    const long long h = hg0 + gh;
    if constexpr (PARTIAL) {
      const long long slot = h * nsplit + split;
      part_o[slot * D + d] = ob;
      if (d == 0) {
        part_ml[2 * slot] = mb;
        part_ml[2 * slot + 1] = lb;
      }
    } else {
      out[h * D + d] = static_cast<_Float16>(lb > 0.0f ? ob / lb : 0.0f);
    }
  }
}

// One query head per KV head (MHA, or GQA sharing switched off) at D = 64 or
// 128 on aligned caches: the wave layout of flash_decode_gqa_wave_kernel --
// NW waves (1, 2, 4 or 8), 32-key blocks (block b of the split to wave
// b % NW) loaded straight into registers with P blocks in flight, no LDS or
// barrier until the waves merge -- with the VALU arithmetic of
// flash_decode_gqa_dma_kernel: LPK = D / 8 lanes hold a key (8 dims each, one
// 16-byte load of K and of V), so one wave load reads KPL = 64 / LPK
// consecutive keys (1 KiB); a score is the v_dot2 of the fp16 q and K pairs
// summed over the key's lanes with DPP. Each of the KPL lane groups keeps its
// own online softmax state (m, l, o of its 8 dims) over the keys it reads, so
// a block needs no exchange between groups; the groups merge once at the end
// (DPP row_ror:8, v_permlane16_swap, v_permlane32_swap: lanes i ^ 8, i ^ 16,
// i ^ 32), then the waves through LDS in wave order.
template <int D, int NW, int P, bool RING, bool PARTIAL>
__global__ __launch_bounds__(64 * NW) void flash_decode_mha_wave_kernel(
    const _Float16* __restrict__ q, const _Float16* k, const _Float16* v,
    _Float16* __restrict__ out, float* __restrict__ part_o, float* __restrict__ part_ml,
    long long kv_len, long long group_size, long long kv_head_stride, float scale, int nsplit) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(NW == 1 || NW == 2 || NW == 4 || NW == 8, "1, 2, 4 or 8 waves");
  static_assert(P >= 1 && P <= 4, "1 to 4 blocks in flight per wave");
  constexpr int LPK = D / 8;                 // lanes per key
  constexpr int KPL = 64 / LPK;              // keys per wave load
  constexpr int KB = 32;                     // keys per block
  constexpr int LPB = KB / KPL;              // loads of K (and of V) per lane per block
  constexpr int WS = D + 2;                  // floats of one wave's state in LDS
  __shared__ __attribute__((aligned(16))) float s_state[NW > 1 ? NW * WS : 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sub = lane / LPK;                // key of a wave load
  const int d0 = (lane % LPK) * 8;           // this lane's dims
  const long long h = blockIdx.x;
  const int split = static_cast<int>(blockIdx.y);
  const long long j0 = kv_len * split / nsplit;
  const long long j1 = kv_len * (split + 1) / nsplit;
  const int nkeys = static_cast<int>(j1 - j0);
  const int nblocks = (nkeys + KB - 1) / KB;
  const int nb = wave < nblocks ? (nblocks - wave + NW - 1) / NW : 0;
  const float scale2 = scale * kLog2e;

  H2 qh[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) qh[p] = H2{q[h * D + d0 + 2 * p], q[h * D + d0 + 2 * p + 1]};

  const long long kvh = h / group_size;
  const _Float16* kb = k + kvh * kv_head_stride + j0 * D + d0;
  const _Float16* vb = v + kvh * kv_head_stride + j0 * D + d0;
  struct Block {
    H8 k[LPB];
    H8 v[LPB];
  };
  // Every call issues the same 2 LPB loads (rows past the split's end read
  // its last key, in bounds, and are masked; a block past the wave's last
  // one is the last key for every lane).
  auto load = [&](Block& b, int t) __attribute__((always_inline)) {
    const int key0 = (wave + NW * t) * KB + sub;
#pragma unroll
    for (int i = 0; i < LPB; ++i) {
      const long long kk = min(key0 + i * KPL, nkeys - 1);
      b.k[i] = __builtin_nontemporal_load(reinterpret_cast<const H8*>(kb + kk * D));
    }
#pragma unroll
    for (int i = 0; i < LPB; ++i) {
      const long long kk = min(key0 + i * KPL, nkeys - 1);
      b.v[i] = __builtin_nontemporal_load(reinterpret_cast<const H8*>(vb + kk * D));
    }
  };

  constexpr float kLazy = 8.0f;              // see flash_decode_gqa_wave_kernel
  float m = kNegInf;
  float l = 0.0f;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;

  auto compute = [&](const Block& b, int t) __attribute__((always_inline)) {
    const int key0 = (wave + NW * t) * KB + sub;
    float sc[LPB];
    float cm = kNegInf;
#pragma unroll
    for (int i = 0; i < LPB; ++i) {
      float part = 0.0f;
#pragma unroll
      for (int p = 0; p < 4; ++p)
        part = __builtin_amdgcn_fdot2(qh[p], H2{b.k[i][2 * p], b.k[i][2 * p + 1]}, part, false);
      part = sum_key_lanes<LPK>(part);
      sc[i] = key0 + i * KPL < nkeys ? part * scale2 : kNegInf;
      cm = fmaxf(cm, sc[i]);
    }
    if (__any(cm > m + kLazy)) {
      const float mn = fmaxf(m, cm);
      const float alpha = merge_weight(m, mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= alpha;
    }
#pragma unroll
    for (int i = 0; i < LPB; ++i) {
      const float p = merge_weight(sc[i], m);
      l += p;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = fmaf(p, static_cast<float>(b.v[i][e]), o[e]);
    }
  };

  Block buf[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    load(buf[i], i);
    __builtin_amdgcn_sched_barrier(0);
  }
  asm volatile("" ::: "memory");
  if constexpr (!RING) {
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (i < nb) compute(buf[i], i);
  } else {
    for (int t = 0; t < nb; t += P) {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        if (t + i < nb) compute(buf[i], t + i);
        load(buf[i], t + i + P);
      }
    }
  }

  // Merge the KPL lane groups of the wave: partner lanes i ^ off hold the same
  // dims for other keys. x + y == y + x, so both lanes of a pair agree.
  auto exchange = [&](float x, int off) __attribute__((always_inline)) -> float {
    if (off == 8) {
      return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
    }
    const unsigned u = __float_as_uint(x);
    const auto r = off == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                             : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const unsigned r0 = r[0];
    const unsigned r1 = r[1];
    return __uint_as_float(r0 == u ? r1 : r0);  // the partner's value
  };
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
    const float mp = exchange(m, off);
    const float lp = exchange(l, off);
    float op[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) op[e] = exchange(o[e], off);
    const float mn = fmaxf(m, mp);
    const float wa = merge_weight(m, mn);
    const float wb = merge_weight(mp, mn);
    l = l * wa + lp * wb;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = o[e] * wa + op[e] * wb;
    m = mn;
  }

  if constexpr (NW == 1) {
    if (sub == 0) {
      if constexpr (PARTIAL) {
        const long long slot = h * nsplit + split;
#pragma unroll
        for (int e = 0; e < 8; ++e) part_o[slot * D + d0 + e] = o[e];
        if (lane == 0) {
          part_ml[2 * slot] = m;
          part_ml[2 * slot + 1] = l;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) out[h * D + d0 + e] = static_cast<_Float16>(l > 0.0f ? o[e] / l : 0.0f);
      }
    }
    return;
  }
  float* const ws = s_state + wave * WS;
  if (sub == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ws[d0 + e] = o[e];
    if (lane == 0) {
      ws[D] = m;
      ws[D + 1] = l;
    }
  }
  __syncthreads();
  for (int d = tid; d < D; d += 64 * NW) {
    float mb = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) mb = fmaxf(mb, s_state[w * WS + D]);
    float lb = 0.0f, ob = 0.0f;
    if (mb > kNegInf) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float wt = merge_weight(s_state[w * WS + D], mb);
        lb = fmaf(s_state[w * WS + D + 1], wt, lb);
        ob = fmaf(s_state[w * WS + d], wt, ob);
      }
    }
    if constexpr (PARTIAL) {
      const long long slot = h * nsplit + split;
      part_o[slot * D + d] = ob;
      if (d == 0) {
        part_ml[2 * slot] = mb;
        part_ml[2 * slot + 1] = lb;
      }
    } else {
      out[h * D + d] = static_cast<_Float16>(lb > 0.0f ? ob / lb : 0.0f);
    }
  }
}

// out[h][d] = sum_s w_s o_s[d] / sum_s w_s l_s with w_s = 2^(m_s - max m).
// One 1024-thread workgroup per head: thread (c, d), c = tid / D, merges the
// states of splits c, c + C, ... (C = 1024 / D) online -- loads issued in
// batches of 8 before they are merged; with at most 256 splits a thread walks
// at most 32 -- and the C slice states then merge in slice order through LDS:
// one pass over the partials, one barrier. (The merge is latency-bound: with
// 256 threads per head it took longer than the split kernel at 128+ splits.)
constexpr int kReduceThreads = 1024;
template <int D>
__global__ __launch_bounds__(kReduceThreads) void flash_decode_reduce_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    _Float16* __restrict__ out, int nsplit) {
  constexpr int C = kReduceThreads / D;
  __shared__ float s_o[C][D];
  __shared__ float s_m[C];
  __shared__ float s_l[C];
  const int tid = threadIdx.x;
  const int c = tid / D;
  const int d = tid - c * D;
  const long long base = static_cast<long long>(blockIdx.x) * nsplit;
  float m = kNegInf, l = 0.0f, o = 0.0f;
  const auto merge = [&](float ms, float ls, float os) {
    const float mn = fmaxf(m, ms);
    if (mn > kNegInf) {
      const float wa = merge_weight(m, mn);
      const float wb = merge_weight(ms, mn);
      l = l * wa + ls * wb;
      o = o * wa + os * wb;
      m = mn;
    }
  };
  if (nsplit <= 2 * C) {
    // One or two states per thread (splits c and c + C), all six loads issued
    // before the first merge and held in registers past it (the asm), so the
    // walk costs one round trip: left to the compiler, the l and o loads sink
    // into merge's branch and each state costs two (TinyLlama at 32 splits:
    // four round trips in a row). A second slot past nsplit re-reads the first.
    const int s0 = c < nsplit ? c : nsplit - 1;
    const int s1 = c + C < nsplit ? c + C : s0;
    float m0 = part_ml[2 * (base + s0)], l0 = part_ml[2 * (base + s0) + 1];
    float o0 = part_o[(base + s0) * D + d];
    float m1 = part_ml[2 * (base + s1)], l1 = part_ml[2 * (base + s1) + 1];
    float o1 = part_o[(base + s1) * D + d];
    asm volatile("" : "+v"(m0), "+v"(l0), "+v"(o0), "+v"(m1), "+v"(l1), "+v"(o1));
    if (c < nsplit) merge(m0, l0, o0);
    if (c + C < nsplit) merge(m1, l1, o1);
  } else {
    // Batches of kBatch states: every load of a batch is issued before the first
    // merge (slots past nsplit re-read the last state and are skipped), so a
    // thread's walk costs one round trip per batch (TinyLlama at 64 splits: 0.6
    // us less per call; at one or two states per thread the plain walk is 0.3-0.9
    // us faster). c is uniform across a wave.
    constexpr int kBatch = 8;
    for (int sp0 = c; sp0 < nsplit; sp0 += kBatch * C) {
      float ms[kBatch], ls[kBatch], os[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int sp = sp0 + i * C;
        const long long slot = base + (sp < nsplit ? sp : nsplit - 1);
        ms[i] = part_ml[2 * slot];
        ls[i] = part_ml[2 * slot + 1];
        os[i] = part_o[slot * D + d];
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (sp0 + i * C >= nsplit) break;
        merge(ms[i], ls[i], os[i]);
      }
    }
  }
  s_o[c][d] = o;
  if (d == 0) {
    s_m[c] = m;
    s_l[c] = l;
  }
  __syncthreads();
  if (tid < D) {
    float mg = kNegInf;
#pragma unroll
    for (int cc = 0; cc < C; ++cc) mg = fmaxf(mg, s_m[cc]);
    float lg = 0.0f, og = 0.0f;
    if (mg > kNegInf) {
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        const float w = merge_weight(s_m[cc], mg);
        lg = fmaf(s_l[cc], w, lg);
        og = fmaf(s_o[cc][tid], w, og);
      }
    }
    out[static_cast<long long>(blockIdx.x) * D + tid] =
        static_cast<_Float16>(lg > 0.0f ? og / lg : 0.0f);
  }
}

// Maximum over the 64 lanes of a wave, in every lane: DPP quad_perm xor-1,
// xor-2, row_half_mirror and row_mirror leave each 16-lane row's maximum in
// all of its lanes; the four rows are then read with v_readlane.
__device__ __forceinline__ float wave_max(float x) {
  const auto step = [](float a, auto ctrl) __attribute__((always_inline)) {
    const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), decltype(ctrl)::value,
                                              0xF, 0xF, false);
    return fmaxf(a, __builtin_bit_cast(float, y));
  };
  x = step(x, std::integral_constant<int, 0xB1>{});
  x = step(x, std::integral_constant<int, 0x4E>{});
  x = step(x, std::integral_constant<int, 0x141>{});
  x = step(x, std::integral_constant<int, 0x140>{});
  const int b = __builtin_bit_cast(int, x);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// The merge for at most MAXS (8, 16, 32 or 64) splits: one wave per head, one
// head per workgroup (a CU streams its loads at a few tens of GB/s, so the
// heads are spread over CUs). Lane s < nsplit loads state s's (m, l); every lane
// loads the D / 64 dims it owns of every state's o -- all loads issued before
// the first is used, one round trip -- then w_s = 2^(m_s - max m) in lane s,
// l = sum_s w_s l_s over the wave (gemv::wave_sum, a fixed order) and
// o[d] = sum_s w_s o_s[d] in split order, w_s read from lane s with
// v_readlane. No LDS and no barrier (the 1024-thread merge below pays one
// barrier and an LDS pass; it stays for more than 64 splits).
template <int D, int MAXS>
__global__ __launch_bounds__(64) void flash_decode_merge_wave_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    _Float16* __restrict__ out, int nsplit) {
  static_assert(MAXS == 8 || MAXS == 16 || MAXS == 32 || MAXS == 64, "8 to 64 splits");
  constexpr int DPL = D / 64;                // dims per lane
  const int lane = threadIdx.x;
  const long long h = blockIdx.x;
  const long long base = h * nsplit;
  const int sl = lane < nsplit ? lane : nsplit - 1;
  const float ms_raw = part_ml[2 * (base + sl)];
  const float ls = part_ml[2 * (base + sl) + 1];
  float os[MAXS][DPL];                       // states past nsplit re-read the last one
#pragma unroll
  for (int sp = 0; sp < MAXS; ++sp) {
    const long long slot = base + (sp < nsplit ? sp : nsplit - 1);
#pragma unroll
    for (int j = 0; j < DPL; ++j) os[sp][j] = part_o[slot * D + lane + 64 * j];
  }
  const float ms = lane < nsplit ? ms_raw : kNegInf;
  const float mx = wave_max(ms);
  const float w = merge_weight(ms, mx);      // 0 past nsplit and for empty states
  const float lw = gemv::wave_sum(w * ls);
  float acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.0f;
#pragma unroll
  for (int sp = 0; sp < MAXS; ++sp) {
    const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), sp));
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = fmaf(ws, os[sp][j], acc[j]);
  }
#pragma unroll
  for (int j = 0; j < DPL; ++j)
    out[h * D + lane + 64 * j] = static_cast<_Float16>(lw > 0.0f ? acc[j] / lw : 0.0f);
}

// Splits when the caller passes split_kv = 0. For flash_decode_gqa_wave_kernel
// (D = 64 GQA on aligned caches): up to 256 keys, one split (one 32-key block
// per wave of an 8-wave workgroup, and no merge launch); longer, 32-key splits
// up to 32 of them, then 512 keys per split (max(min(L / 32, 32), L / 512)),
// at most one workgroup per CU over all head groups. A sweep on MI355X at
// TinyLlama's 32 / 4 heads (4 head groups), cold caches, 1 to 128 splits, put
// this at the best split count or within 1.5% of it for 128 to 32768 keys
// (e.g. 512 keys: 16 splits, 5.15 us; 2048: 32, 6.4 us; 32768: 64, 11.3 us).
// For the other kernels: about one workgroup per CU, at least 64 keys per
// split, at most 256 splits (the same kind of sweep over 32 / 4 heads at
// D = 64 and 32 / 32 at D = 128, 512 to 32768 keys).
int auto_splits(long long kv_len, long long head_blocks, bool wave_kernel) {
  const long long cus = device_cu_count();
  if (wave_kernel) {
    if (kv_len <= 256) return 1;
    const long long s = std::max(std::min(kv_len / 32, 32LL), kv_len / 512);
    return static_cast<int>(std::max(1LL, std::min({s, std::max(1LL, cus / head_blocks), 256LL})));
  }
  const long long wanted = (cus + head_blocks - 1) / head_blocks;
  const long long by_len = kv_len / 64;
  return static_cast<int>(std::max(1LL, std::min({wanted, by_len, 256LL})));
}

struct DecodeArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  _Float16* out;
  long long kv_len, n_heads, group_size, kv_head_stride;
  float scale;
  int splits;
};

// 16-byte aligned caches: GQA groups on flash_decode_gqa_wave_kernel (matrix
// cores, K / V straight into registers), one head per workgroup (MHA, or GQA
// sharing switched off) on flash_decode_mha_wave_kernel (VALU, K / V straight
// into registers), long D = 64 single-head splits on the direct-to-LDS
// pipelined kernel. Unaligned caches: one query
// head per workgroup on the register kernel with 8 key steps in flight per
// lane; GQA groups on the register-staged LDS-tile kernel.

// flash_decode_gqa_wave_kernel's shape from the longest split's 32-key
// blocks: up to 8 blocks, one wave per block (1, 2, 4 or 8 waves, so a
// one-block split is one wave with no LDS merge); more, 8 waves with every
// block in flight at once (2 or 4 per wave) or a ring of 4.
template <int D, int G, bool PARTIAL>
void launch_wave(const DecodeArgs& a, float* part_o, float* part_ml, dim3 grid, hipStream_t s) {
  // A block is 2 D bytes per lane in registers: up to 4 in flight at D = 64,
  // 2 at D = 128.
  constexpr int PMAX = D == 64 ? 4 : 2;
  const long long keys = (a.kv_len + a.splits - 1) / a.splits;
  const long long blocks = (keys + 31) / 32;
  auto go = [&](auto kernel, int waves) {
    kernel<<<grid, 64 * waves, 0, s>>>(a.q, a.k, a.v, a.out, part_o, part_ml, a.kv_len,
                                       a.group_size, a.kv_head_stride, a.scale, a.splits);
  };
  if (blocks <= 1) {
    go(flash_decode_gqa_wave_kernel<D, G, 1, 1, false, PARTIAL>, 1);
  } else if (blocks <= 2) {
    go(flash_decode_gqa_wave_kernel<D, G, 2, 1, false, PARTIAL>, 2);
  } else if (blocks <= 4) {
    go(flash_decode_gqa_wave_kernel<D, G, 4, 1, false, PARTIAL>, 4);
  } else if (blocks <= 8) {
    go(flash_decode_gqa_wave_kernel<D, G, 8, 1, false, PARTIAL>, 8);
  } else if (blocks <= 16) {
    go(flash_decode_gqa_wave_kernel<D, G, 8, 2, false, PARTIAL>, 8);
  } else if (PMAX == 4 && blocks <= 32) {
    go(flash_decode_gqa_wave_kernel<D, G, 8, PMAX, false, PARTIAL>, 8);
  } else {
    go(flash_decode_gqa_wave_kernel<D, G, 8, PMAX, true, PARTIAL>, 8);
  }
}

template <int D, bool PARTIAL>
void launch_mha_wave(const DecodeArgs& a, float* part_o, float* part_ml, dim3 grid, hipStream_t s) {
  const long long keys = (a.kv_len + a.splits - 1) / a.splits;
  const long long blocks = (keys + 31) / 32;
  auto go = [&](auto kernel, int waves) {
    kernel<<<grid, 64 * waves, 0, s>>>(a.q, a.k, a.v, a.out, part_o, part_ml, a.kv_len,
                                       a.group_size, a.kv_head_stride, a.scale, a.splits);
  };
  constexpr int PMAX = D == 64 ? 4 : 2;      // 32 (64) VGPRs per block at D = 64 (128)
  if (blocks <= 1) {
    go(flash_decode_mha_wave_kernel<D, 1, 1, false, PARTIAL>, 1);
  } else if (blocks <= 2) {
    go(flash_decode_mha_wave_kernel<D, 2, 1, false, PARTIAL>, 2);
  } else if (blocks <= 4) {
    go(flash_decode_mha_wave_kernel<D, 4, 1, false, PARTIAL>, 4);
  } else if (blocks <= 8) {
    go(flash_decode_mha_wave_kernel<D, 8, 1, false, PARTIAL>, 8);
  } else if (blocks <= 16) {
    go(flash_decode_mha_wave_kernel<D, 8, 2, false, PARTIAL>, 8);
  } else if (blocks <= 8 * PMAX) {
    go(flash_decode_mha_wave_kernel<D, 8, PMAX, false, PARTIAL>, 8);
  } else {
    go(flash_decode_mha_wave_kernel<D, 8, PMAX, true, PARTIAL>, 8);
  }
}

template <int D, int G, bool VEC, bool PARTIAL>
void launch_split(const DecodeArgs& a, float* part_o, float* part_ml, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.n_heads / G), static_cast<unsigned>(a.splits));
  if constexpr (VEC && G >= 2) {
    launch_wave<D, G, PARTIAL>(a, part_o, part_ml, grid, s);
  } else if constexpr (VEC) {
    // One head per workgroup: the register-fed kernel, except at D = 64 for
    // splits past 8 waves x 4 blocks (its ring streamed a TinyLlama head without
    // GQA sharing, 4096-key splits, at 5.7 TB/s; the LDS pipeline at 6.3).
    const long long blocks = ((a.kv_len + a.splits - 1) / a.splits + 31) / 32;
    if (G == 1 && (D == 128 || blocks <= 32)) {
      launch_mha_wave<D, PARTIAL>(a, part_o, part_ml, grid, s);
    } else {
      flash_decode_gqa_dma_kernel<D, G, PARTIAL><<<grid, kThreads, 0, s>>>(
          a.q, a.k, a.v, a.out, part_o, part_ml, a.kv_len, a.group_size, a.kv_head_stride,
          a.scale, a.splits);
    }
  } else if constexpr (G == 1) {
    flash_decode_split_kernel<D, 1, 8, VEC, PARTIAL><<<grid, kThreads, 0, s>>>(
        a.q, a.k, a.v, a.out, part_o, part_ml, a.kv_len, a.group_size, a.kv_head_stride,
        a.scale, a.splits);
  } else {
    flash_decode_gqa_lds_kernel<D, G, VEC, PARTIAL><<<grid, kThreads, 0, s>>>(
        a.q, a.k, a.v, a.out, part_o, part_ml, a.kv_len, a.group_size, a.kv_head_stride,
        a.scale, a.splits);
  }
  ENG_LAUNCH_CHECK();
}

template <int D, int G, bool VEC>
void run_decode(const DecodeArgs& a, hipStream_t s) {
  if (a.splits == 1) {
    launch_split<D, G, VEC, false>(a, nullptr, nullptr, s);
    return;
  }
  const std::size_t slots = static_cast<std::size_t>(a.n_heads) * a.splits;
  StreamScratch scratch(s, slots * (D + 2) * sizeof(float));
  float* part_o = static_cast<float*>(scratch.get());
  float* part_ml = part_o + slots * D;
  launch_split<D, G, VEC, true>(a, part_o, part_ml, s);
  const unsigned heads = static_cast<unsigned>(a.n_heads);
  if (a.splits <= 8) {
    flash_decode_merge_wave_kernel<D, 8><<<heads, 64, 0, s>>>(part_o, part_ml, a.out, a.splits);
  } else if (a.splits <= 16) {
    flash_decode_merge_wave_kernel<D, 16><<<heads, 64, 0, s>>>(part_o, part_ml, a.out, a.splits);
  } else if (a.splits <= 32) {
    flash_decode_merge_wave_kernel<D, 32><<<heads, 64, 0, s>>>(part_o, part_ml, a.out, a.splits);
  } else if (a.splits <= 64) {
    flash_decode_merge_wave_kernel<D, 64><<<heads, 64, 0, s>>>(part_o, part_ml, a.out, a.splits);
  } else {
    flash_decode_reduce_kernel<D><<<static_cast<unsigned>(a.n_heads), kReduceThreads, 0, s>>>(
        part_o, part_ml, a.out, a.splits);
  }
  ENG_LAUNCH_CHECK();
}

template <int D, bool VEC>
void run_decode_g(const DecodeArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 8: run_decode<D, 8, VEC>(a, s); break;
    case 4: run_decode<D, 4, VEC>(a, s); break;
    case 2: run_decode<D, 2, VEC>(a, s); break;
    default: run_decode<D, 1, VEC>(a, s); break;
  }
}

void attention_decode_any(const eng_half* q, const eng_half* k, const eng_half* v, eng_half* out,
                          int64_t kv_len, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                          int64_t kv_head_stride, float scale, int split_kv, bool share_gqa_kv,
                          eng_stream stream) {
  // Precondition order and messages: reference kernels/attention_decode.cu:590-607.
  ENG_CHECK(q != nullptr, "attention_decode: q is null");
  ENG_CHECK(k != nullptr, "attention_decode: k is null");
  ENG_CHECK(v != nullptr, "attention_decode: v is null");
  ENG_CHECK(out != nullptr, "attention_decode: out is null");
  ENG_CHECK(kv_len >= 0, "attention_decode: kv_len must be non-negative");
  ENG_CHECK(n_heads > 0, "attention_decode: n_heads must be positive");
  ENG_CHECK(n_kv_heads > 0, "attention_decode: n_kv_heads must be positive");
  ENG_CHECK(n_heads % n_kv_heads == 0,
            "attention_decode: n_heads must be divisible by n_kv_heads");
  ENG_CHECK(head_dim == 64 || head_dim == 128, "attention_decode: head_dim must be 64 or 128");
  ENG_CHECK(std::isfinite(scale), "attention_decode: scale must be finite");
  ENG_CHECK(split_kv >= 0, "attention_decode: split_kv must be non-negative");
  const int64_t min_stride = kv_len > 0 ? kv_len * head_dim : 0;
  ENG_CHECK(kv_head_stride >= min_stride,
            "attention_decode: kv_head_stride < kv_len * head_dim");
  hipStream_t s = as_stream(stream);
  if (kv_len == 0) {
    fill_zero_async(out, static_cast<std::size_t>(n_heads * head_dim) * sizeof(eng_half), s);
    return;
  }
  ENG_CHECK(n_heads <= 0x7fffffffLL, "attention_decode: n_heads too large for one launch");

  DecodeArgs a;
  a.q = reinterpret_cast<const _Float16*>(q);
  a.k = reinterpret_cast<const _Float16*>(k);
  a.v = reinterpret_cast<const _Float16*>(v);
  a.out = reinterpret_cast<_Float16*>(out);
  a.kv_len = kv_len;
  a.n_heads = n_heads;
  a.group_size = n_heads / n_kv_heads;
  a.kv_head_stride = kv_head_stride;
  a.scale = scale;
  // Query heads per workgroup: the largest of 8, 4, 2 dividing the GQA group
  // when K / V are shared across it, otherwise one.
  int G = 1;
  if (share_gqa_kv) {
    for (int cand : {8, 4, 2}) {
      if (a.group_size % cand == 0) {
        G = cand;
        break;
      }
    }
  }
  // Explicit requests are clamped to kv_len (as the reference does) and to
  // 256 (more splits only add partial states to merge); the result does not
  // depend on the split count beyond rounding.
  const bool vec = aligned_to(k, 16) && aligned_to(v, 16) && kv_head_stride % 8 == 0;
  const bool wave_kernel = vec && G >= 2;
  const int req = split_kv == 0 ? auto_splits(kv_len, n_heads / G, wave_kernel) : split_kv;
  a.splits = static_cast<int>(std::max<long long>(1, std::min<long long>({req, kv_len, 256})));
  if (head_dim == 64) {
    if (vec) {
      run_decode_g<64, true>(a, G, s);
    } else {
      run_decode_g<64, false>(a, G, s);
    }
  } else {
    if (vec) {
      run_decode_g<128, true>(a, G, s);
    } else {
      run_decode_g<128, false>(a, G, s);
    }
  }
}

// ------------------------------------------------------------------ bridge
__global__ __launch_bounds__(kThreads) void cast_f32_to_f16_kernel(const float* __restrict__ in,
                                                                   _Float16* __restrict__ out,
                                                                   long long n) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    out[i] = static_cast<_Float16>(in[i]);
  }
}

__global__ __launch_bounds__(kThreads) void cast_f16_to_f32_kernel(const _Float16* __restrict__ in,
                                                                   float* __restrict__ out,
                                                                   long long n) {
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    out[i] = static_cast<float>(in[i]);
  }
}

// Token-major new K / V [s_new, n_kv_heads, D] -> head-major caches
// [n_kv_heads, kv_max_seq_len, D] at positions pos_offset ...
__global__ __launch_bounds__(kThreads) void kv_cache_write_kernel(
    const _Float16* __restrict__ k_new, const _Float16* __restrict__ v_new,
    _Float16* __restrict__ k_cache, _Float16* __restrict__ v_cache, long long s_new,
    long long n_kv_heads, long long D, long long pos_offset, long long kv_max_seq_len) {
  const long long total = s_new * n_kv_heads * D;
  const long long stride = static_cast<long long>(gridDim.x) * kThreads;
  for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += stride) {
    const long long d = i % D;
    const long long th = i / D;
    const long long h = th % n_kv_heads;
    const long long t = th / n_kv_heads;
    const long long dst = (h * kv_max_seq_len + pos_offset + t) * D + d;
    k_cache[dst] = k_new[i];
    v_cache[dst] = v_new[i];
  }
}

unsigned bridge_grid(long long n) {
  const long long wanted = 8LL * device_cu_count();
  return static_cast<unsigned>(std::max(1LL, std::min((n + kThreads - 1) / kThreads, wanted)));
}

}  // namespace
}  // namespace eng

using eng::guarded;

extern "C" {

int eng_attention_decode_f16(const eng_half* q, const eng_half* k, const eng_half* v,
                             eng_half* out, int64_t kv_len, int64_t n_heads, int64_t n_kv_heads,
                             int64_t head_dim, int64_t kv_head_stride, float scale, int split_kv,
                             eng_stream stream) {
  return guarded([&] {
    eng::attention_decode_any(q, k, v, out, kv_len, n_heads, n_kv_heads, head_dim,
                              kv_head_stride, scale, split_kv, true, stream);
  });
}

int eng_attention_decode_with_mode_f16(const eng_half* q, const eng_half* k, const eng_half* v,
                                       eng_half* out, int64_t kv_len, int64_t n_heads,
                                       int64_t n_kv_heads, int64_t head_dim,
                                       int64_t kv_head_stride, float scale, int split_kv,
                                       int share_gqa_kv, eng_stream stream) {
  return guarded([&] {
    eng::attention_decode_any(q, k, v, out, kv_len, n_heads, n_kv_heads, head_dim,
                              kv_head_stride, scale, split_kv, share_gqa_kv != 0, stream);
  });
}

int eng_cast_f32_to_f16(const float* in, eng_half* out, int64_t n, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(n >= 0, "cast_f32_to_f16: n must be non-negative");
    if (n == 0) return;
    ENG_CHECK(in != nullptr, "cast_f32_to_f16: in is null");
    ENG_CHECK(out != nullptr, "cast_f32_to_f16: out is null");
    eng::cast_f32_to_f16_kernel<<<eng::bridge_grid(n), eng::kThreads, 0, eng::as_stream(stream)>>>(
        in, reinterpret_cast<_Float16*>(out), n);
    ENG_LAUNCH_CHECK();
  });
}

int eng_cast_f16_to_f32(const eng_half* in, float* out, int64_t n, eng_stream stream) {
  return guarded([&] {
    ENG_CHECK(n >= 0, "cast_f16_to_f32: n must be non-negative");
    if (n == 0) return;
    ENG_CHECK(in != nullptr, "cast_f16_to_f32: in is null");
    ENG_CHECK(out != nullptr, "cast_f16_to_f32: out is null");
    eng::cast_f16_to_f32_kernel<<<eng::bridge_grid(n), eng::kThreads, 0, eng::as_stream(stream)>>>(
        reinterpret_cast<const _Float16*>(in), out, n);
    ENG_LAUNCH_CHECK();
  });
}

int eng_kv_cache_write_f16(const eng_half* k_new, const eng_half* v_new, eng_half* k_cache,
                           eng_half* v_cache, int64_t s_new, int64_t n_kv_heads, int64_t head_dim,
                           int64_t pos_offset, int64_t kv_max_seq_len, eng_stream stream) {
  return guarded([&] {
    // Precondition order and messages: reference kernels/attention_bridge.cu:86-103.
    ENG_CHECK(s_new >= 0, "kv_cache_write: s_new must be non-negative");
    ENG_CHECK(n_kv_heads > 0, "kv_cache_write: n_kv_heads must be positive");
    ENG_CHECK(head_dim > 0, "kv_cache_write: head_dim must be positive");
    ENG_CHECK(pos_offset >= 0, "kv_cache_write: pos_offset must be non-negative");
    ENG_CHECK(kv_max_seq_len >= pos_offset + s_new,
              "kv_cache_write: kv_max_seq_len < pos_offset + s_new");
    if (s_new == 0) return;
    ENG_CHECK(k_new != nullptr && v_new != nullptr, "kv_cache_write: k_new/v_new is null");
    ENG_CHECK(k_cache != nullptr && v_cache != nullptr, "kv_cache_write: k_cache/v_cache is null");
    const long long total = s_new * n_kv_heads * head_dim;
    eng::kv_cache_write_kernel<<<eng::bridge_grid(total), eng::kThreads, 0,
                                 eng::as_stream(stream)>>>(
        reinterpret_cast<const _Float16*>(k_new), reinterpret_cast<const _Float16*>(v_new),
        reinterpret_cast<_Float16*>(k_cache), reinterpret_cast<_Float16*>(v_cache), s_new,
        n_kv_heads, head_dim, pos_offset, kv_max_seq_len);
    ENG_LAUNCH_CHECK();
  });
}

}  // extern "C"
