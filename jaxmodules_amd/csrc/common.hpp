// Shared definitions of the gfx950 masked-attention kernels.
//
// Tile vocabulary (all kernels):
//   * map tile   : 128 queries x 128 keys, the granularity of the block map
//                  (mattn_blockmap in include/mattn.h);
//   * sub-block  : 64 keys (forward, dQ) or 64 queries (dK/dV), the unit one
//                  pipeline stage stages through LDS;
//   * MFMA tile  : 32 x 32 outputs of v_mfma_f32_32x32x16_{bf16,f16}.
//
// MFMA 32x32x16 operand layout (lane l, l32 = l % 32, hi = l / 32):
//   A[32 x 16]: lane holds row l32, k = 8*hi .. 8*hi+7   (16 contiguous bytes)
//   B[16 x 32]: lane holds col l32, k = 8*hi .. 8*hi+7
//   C[32 x 32]: lane holds col l32, register r holds row 8*(r/4) + 4*hi + r%4
// A C-tile's registers [8*j, 8*j+8) of lane (l32, hi) therefore cover rows
// 16*j + {0..3, 8..11} (hi = 0) or 16*j + {4..7, 12..15} (hi = 1): exactly
// the 8 values a B (or A) operand of the next product needs for a 16-deep
// k-step, provided the matching operand is read with the same row
// permutation: the transposed operand reads (two ds_read_b64_tr_b16 of 4
// rows each, tr_src) fetch rows {4 hi .. 4 hi + 3} and {8 + 4 hi .. 8 + 4 hi
// + 3} of the k-step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <utility>

#include "mattn.h"

namespace mattn {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int TILE = 128;  // map tile edge (MATTN_TILE_Q == MATTN_TILE_K)
constexpr float NEG_INF = -__builtin_inff();

// Arguments of every kernel (passed by value in the kernarg segment).
//
// The 16-bit paths multiply float16 operands only.  Every float16 working copy
// is the input times a power of two per 128-row tile (copy_scale: exact for
// bfloat16 and float16 values), written head-major and dense,
// [B, H, rows padded to 128, D], rows past the sequence end zero:
//   vh = V * vsc[b, hk, key tile]    qh  = Q * qsc[b, h, query tile]   (forward)
//   kh = K * ksc[b, hk, key tile]    doh = dO * dsc[b, h, query tile]  (backward)
// so each product's scale is a per-step scalar, undone on the float32 result.
// The forward leaves vh and qh (with their scales) for the backward.
struct KArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;     // forward output (read by the backward preprocess)
  const void* dO;    // upstream gradient in o_dtype
  void* out;         // forward output O
  float* lse;        // [B, Hq, Lq] base-2 log-sum-exp
  float* delta;      // [B, Hq, Lq] rowsum(O * doh): delta in units of dsc
  void* dq;
  void* dk;
  void* dv;
  uint16_t* vh;      // [B, Hkv, nkt*128, D] (forward residual)
  uint16_t* qh;      // [B, Hq, nqt*128, D] (forward residual; the forward writes it when non-null)
  uint16_t* kh;      // [B, Hkv, nkt*128, D] (backward)
  uint16_t* doh;     // [B, Hq, nqt*128, D] (backward)
  float* vsc;        // [B*Hkv*nkt] scale of each V tile
  float* vmax;       // [B*Hkv*nkt] max |V| of each tile
  float* qsc;        // [B*Hq*nqt] scale of each Q tile
  float* ksc;        // [B*Hkv*nkt] scale of each K tile
  float* dsc;        // [B*Hq*nqt] scale of each dO tile
  float2* tst;       // [B*Hq*nqt] per query tile: (max row L1 norm of doh, max |delta|)
  float* asc;        // [B*Hq*nqt] per query tile: f * dsc, f the dK/dV kernel's dS scale
  float* lsf;        // [B, Hq, Lq] lse - log2(f) of the row's tile (the dK/dV kernel's P * f)
  int64_t qs[3], ks[3], vs[3], os[3], dos[3], dqs[3], dks[3], dvs[3];
  int B, Lq, Lk, Hq, Hkv, G;
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
  int map_b, map_h, nqt, nkt;
  const int* row_ptr;
  const int* row_ent;
  const int* col_ptr;
  const int* col_ent;
  const uint64_t* row_bits;
  const uint64_t* col_bits;
  const int* q_order;
  const int* kv_order;
  // MATTN_BWD_DS: dS fragments of every present tile (null: dQ recomputes dS);
  // slot of tile e (row-entry index) of (b, h): rep * ds_nnz + e, where rep
  // counts the (b, h) that share the map's entries
  uint16_t* ds;
  const int* col_row;
  int ds_nnz;
  const int* kv_desc;  // per dK/dV launch slot: { item, g, e, e_end, n_sub, qt, mask, row }
  int precise;         // MATTN_PRECISE: the SIMT kernels form the scores as compensated dot products
  float* lse_lo;       // MATTN_PRECISE (SIMT, forward residual): [B, Hq, Lq], (m + log2 l) - lse
  float* o_lo;         // MATTN_PRECISE (SIMT, forward residual): [B, Hq, Lq, D], exact O - stored O
  // Split rows (MFMA path): a row whose largest attention weight reaches
  // SPLIT_P.  The forward leaves per query tile the largest weight of its
  // rows (pmx) and a 128-bit mask of its split rows (srow, 4 words, bit i of
  // word w = row 32 w + i); a tile with a split row is a split tile.  bwd_pre
  // stores the part of dO' that float16 rounds off in a split tile's rows
  // (dol, [B, Hq, nqt*128, D]), takes the split rows' delta from the
  // unrounded dO and marks the tile by a negative asc; kernels of their own
  // then form the split rows' O, lse and dQ, and the dK / dV terms of the
  // split rows' allowed pairs, with the products of those rounded-off parts
  // (of dO', P and dS): 22 significant bits instead of 11.
  float* pmx;
  uint32_t* srow;
  uint16_t* dol;
  int* scol;           // [B*Hkv*nkt] per dK/dV column: a split row has an allowed key in it
  float* kvp;          // [B*Hkv*nkt][2][128][D] such a column's unrounded dK, dV (units of 1)
};

// Largest attention weight from which a query tile is a split tile.  Rows
// whose weights are all below it put each key's gradient terms on many
// queries, whose float16 rounding errors average out below the parity
// gate's float32-accumulation slack; rows with a dominant key do not (a
// bfloat16 gradient one ulp off where the exact value lies near a rounding
// midpoint).
constexpr float SPLIT_P = 0.03125f;

// dS storage slot base of (b, h): the map's entries are shared by the (b, h)
// it broadcasts over, each of which has slots of its own
__device__ __forceinline__ int64_t ds_rep(const KArgs& a, int b, int h) {
  const int rb = a.map_b == 1 ? b : 0, rh = a.map_h == 1 ? h : 0;
  return ((int64_t)rb * (a.map_h == 1 ? a.Hq : 1) + rh) * a.ds_nnz;
}
// Row walks of the split kernels (forward, dQ): of the first 64 entries of
// map row [e0, e1) of query tile `item`, those where a split row of the tile
// has an allowed key (a full tile, or a mask word of a split row not zero),
// as a bit mask (entries past the first 64 always count).  Every wave finds
// the same mask: lane l checks rows l and l + 64 (the words of the mask id
// met last are reused, as the entries of a row often share one).
// (sr0, sr1: the split-row words of the waves whose rows are lane and lane + 64)
__device__ __forceinline__ uint64_t split_entries_w(const KArgs& a, uint32_t sr0, uint32_t sr1, int e0, int e1,
                                                    int lane) {
  const bool s0 = (sr0 >> (lane & 31)) & 1u, s1 = (sr1 >> (lane & 31)) & 1u;
  const int n64 = min(e1 - e0, 64);
  const int mk = a.row_ent[2 * min(e0 + lane, e1 - 1) + 1];
  uint64_t need = 0ull;
  int last = -2;
  bool last_need = true;
  for (int i = 0; i < n64; ++i) {
    const int m = __builtin_amdgcn_readlane(mk, i);
    if (m != last) {
      last = m;
      if (m < 0) {
        last_need = true;
      } else {
        const uint64_t* w = a.row_bits + (int64_t)m * 2 * TILE;
        const bool hit = (s0 && (w[lane] | w[TILE + lane]) != 0) || (s1 && (w[64 + lane] | w[TILE + 64 + lane]) != 0);
        last_need = __any(hit);
      }
    }
    if (last_need) need |= 1ull << i;
  }
  return need;
}
__device__ __forceinline__ uint64_t split_entries(const KArgs& a, int item, int e0, int e1, int lane) {
  return split_entries_w(a, a.srow[item * 4 + (lane >> 5)], a.srow[item * 4 + 2 + (lane >> 5)], e0, e1, lane);
}
// The entry after `e` that split_entries counts (e0 - 1 for the first).
__device__ __forceinline__ int split_next(uint64_t need, int e, int e0) {
  const int i = e + 1 - e0;
  if (i >= 64) return e + 1;
  const uint64_t rest = need >> i;
  return rest ? e + 1 + (int)__builtin_ctzll(rest) : e0 + 64;
}
// Sub-blocks (two per entry) of such a walk.
__device__ __forceinline__ int split_subblocks(uint64_t need, int e0, int e1) {
  return 2 * (__builtin_popcountll(need) + max(e1 - e0 - 64, 0));
}

// Elements of one tile's dS (128 x 128 float16), as the dK/dV kernel's waves
// hold it (lane = key): per 32-query group w, 32-key group kg and 16-query
// half t, a 1 KiB block at (8 w + 2 kg + t) * 512 elements of 64 16-byte
// chunks.  Chunk of lane l (key 32 kg + l % 32, hi = l / 32) = queries
// 32 w + 16 t + 4 hi + 8 j + i (j = 0, 1; i = 0..3) in slots 4 j + i, stored
// at position ds_pos(l, t) of the block.  The permutation makes the dQ
// kernel's transposed 8-byte reads of a block (4 keys x 16 queries per
// 16 lanes) hit 32 distinct bank pairs per 32 lanes.
constexpr int DS_TILE = TILE * TILE;
__device__ __forceinline__ int ds_pos(int l, int t) { return l ^ ((((l >> 5) & 1) << 2) | (t << 3)); }

// Power of two s with m * s in [2^(top-1), 2^top) for finite m > 0 (1 otherwise).
__device__ __forceinline__ float pow2_scale(float m, int top) {
  if (!(m > 0.f) || !(m <= 3.4e38f)) return 1.f;
  int e;
  frexpf(m, &e);  // m in [2^(e-1), 2^e)
  return ldexpf(1.f, min(126, max(-126, top - e)));
}

// Scale of a float16 working copy from the largest magnitude m it holds: a
// power of two s with m * s in [2^10, 2^14), s's exponent a multiple of 4.
// Copies whose maxima lie within a factor of 16 of each other then mostly get
// the same s, so the kernels rarely rescale an accumulator between tiles.  A
// bfloat16 value is exact in float16 down to 2^-17 (and a float32 value keeps
// 11 significant bits down to 2^-14), i.e. to 2^-27 of the copy's maximum.
__device__ __forceinline__ float copy_scale(float m) {
  if (!(m > 0.f) || !(m <= 3.4e38f)) return 1.f;
  int e;
  frexpf(m, &e);                           // m in [2^(e-1), 2^e)
  const int t = (e + 3 + 256) / 4 * 4 - 256;  // e rounded up to a multiple of 4
  return ldexpf(1.f, min(124, max(-124, 14 - t)));
}

// Scale f of a query tile's float16 dS in the dK/dV kernel: |dS| <= bound (in
// the units dS is computed in) keeps |dS * f| < 2^14; f's exponent is a
// multiple of 4 (tiles then mostly share it, as with copy_scale) and at most
// 12, so that f * P (P <= 1) stays inside float16 too.
__device__ __forceinline__ float ds_scale(float bound) {
  if (!(bound > 0.f) || !(bound <= 3.4e38f)) return 4096.f;
  int e;
  frexpf(bound, &e);                          // bound in [2^(e-1), 2^e)
  const int k = (14 - e + 256) / 4 * 4 - 256;  // floor((14 - e) / 4) * 4
  return ldexpf(1.f, min(12, max(-124, k)));
}

// 1 / x for a power of two x = 2^k, |k| <= 126: exact (exponent arithmetic).
__device__ __forceinline__ float pow2_rcp(float x) {
  return __uint_as_float(0x7f000000u - __float_as_uint(x));
}

struct bf16_tag {};
struct f16_tag {};

template <class Tag>
struct Elt;

template <>
struct Elt<bf16_tag> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32)
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  }
  static __device__ __forceinline__ float to_f32(uint32_t bits16) {
    return __builtin_bit_cast(float, bits16 << 16);
  }
};

template <>
struct Elt<f16_tag> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
  static __device__ __forceinline__ float to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16-bit element j (0..7) of a 16-byte chunk.
__device__ __forceinline__ uint32_t elt16(const u32x4& x, int j) {
  return (x[j >> 1] >> ((j & 1) * 16)) & 0xffffu;
}

// LDS layouts.  gfx950 LDS has 64 banks of 4 bytes: a ds_read_b128 serves 16
// lanes per cycle, a ds_write_b64 32 lanes, so a 16-lane group must touch 16
// distinct 16-byte bank groups.
//
// Row-major tile [rows][D] of 16-bit values, rows packed, filled by direct
// global->LDS loads.  The 16-byte chunk c of row r is stored at chunk
// c ^ swz<D>(r).  The swizzle makes both operand access patterns
// conflict-free on the 64 banks:
//   * ds_read_b128 row reads: 16 lanes read rows r0..r0+15 at one chunk;
//   * ds_read_b64_tr_b16 reads: 32 lanes read rows r0..r0+3 (r0 % 4 == 0)
//     at 4 consecutive chunks.
// D = 128 (a row spans all banks): swz = 4 (r % 4) + (r / 4) % 4.
// D = 64 (two rows per bank line, row parity picks the half):
// swz = 4 ((r / 2) % 2) + (r / 4) % 4.
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}
template <int D>
__device__ __forceinline__ int sw_off(int r, int c) {  // element offset of chunk c of row r
  return r * D + ((c ^ swz<D>(r)) << 3);
}

// Direct global->LDS tile loader: one global_load_lds_dwordx4 moves 1 KiB
// (64 lanes x 16 bytes, lane L to LDS byte 16 L of the instruction's block).
// Lane L of instruction block n covers row n * RPI + L / CPR of the tile and
// physical chunk L % CPR, i.e. logical chunk (L % CPR) ^ swz(row).
template <int D>
struct TileLoad {
  static constexpr int CPR = D / 8;          // chunks per row
  static constexpr int RPI = 64 / CPR;       // rows per load instruction
  // element offset (row-relative to the tile's first row, stride rs) of
  // lane L's source in instruction block n
  static __device__ __forceinline__ uint32_t src_off(int n, int lane, int64_t rs) {
    const int r = n * RPI + lane / CPR;
    const int c = (lane % CPR) ^ swz<D>(r);
    return (uint32_t)(r * rs + 8 * c);
  }
  static __device__ __forceinline__ int row_of(int n, int lane) { return n * RPI + lane / CPR; }
  static __device__ __forceinline__ int chunk_of(int n, int lane) {
    const int r = n * RPI + lane / CPR;
    return (lane % CPR) ^ swz<D>(r);
  }
};

__device__ __forceinline__ void lds_load16(const void* g, uint16_t* lds_block) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_block, 16, 0, 0);
}

// Buffer resource of `bytes` bytes at `base` (raw, no stride; loads past the
// end return zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Direct global->LDS load of 16 bytes per lane through a buffer resource: lane L
// reads rsrc + soff + voff and lands at lds_block + 16 L (as lds_load16).  The
// address is formed by the load unit: a loop-invariant per-lane voff and a
// uniform soff need no per-load VALU arithmetic.
__device__ __forceinline__ void lds_load16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                               uint16_t* lds_block) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_block, 16, (int)voff,
                                          (int)soff, 0, 0);
}

// Transposed operand read (ds_read_b64_tr_b16, ds_read_tr8 below): inside
// each 16-lane group, if lane j addresses X[r + j/4][c + 4 (j % 4)], lane i
// receives X[r + k][c + i] for k = 0..3.
//
// Element offset, within a swizzled [rows][D] tile, of the address lane
// `lane` supplies to that read so that it receives the A operand
// A[i = 32 mt + lane % 32][k = rows 16 ks + 4 hi + 8 sec + 0..3] of a
// 32x32x16 MFMA k-step (sec = 0: operand slots 0-3, sec = 1: slots 4-7),
// i.e. X[16 ks + 8 sec + 4 hi + k][32 mt + lane % 32].  Returned for ks = 0;
// k-step ks adds 16 * ks * D elements.
template <int D>
__device__ __forceinline__ int tr_src(int lane, int mt, int sec) {
  const int i = lane & 15, g = lane >> 4, hi = lane >> 5;
  const int r = 4 * hi + 8 * sec + (i >> 2);
  const int c = 4 * mt + 2 * (g & 1) + ((i & 3) >> 1);
  return r * D + ((c ^ swz<D>(r)) << 3) + 4 * (i & 1);
}

// Bit of a 64-bit tile-mask word for C-register r of MFMA row tile t (rows
// 32t + 8(r/4) + 4hi + r%4), w32 being the word's half for t pre-shifted by
// 4hi, as all ones (set) or zero (clear): one v_bfe_i32, after which masking
// an element is one v_and_b32 (to 0) or bit-select (to -inf) instead of a
// compare and a select
__device__ __forceinline__ uint32_t mask_ones(uint32_t w32, int r) {
  uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)w32, 8 * (r >> 2) + (r & 3), 1);
  // opaque to the compiler, which would otherwise turn the AND back into a
  // compare and a select (and an s_nop for the VCC hazard between them)
  asm("" : "+v"(m));
  return m;
}
__device__ __forceinline__ float mask_zero(float x, uint32_t m) {
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) & m);
}
__device__ __forceinline__ float mask_neg_inf(float x, uint32_t m) {
  return __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, x) & m) | (~m & 0xff800000u));
}

// max / sum of x over lanes l and l ^ 32 (v_permlane32_swap: no LDS access, so
// no wait on outstanding global->LDS loads)
__device__ __forceinline__ float wave_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Tile-map entries of one map row/column, 64 at a time, one per lane: read
// back with v_readlane at a wave-uniform index (no memory access inside the
// loop, so no wait on the global->LDS loads in flight).  ent holds
// (tile, mask id) pairs; [e0, e1) is the range this workgroup walks.
// Tile entries of one CSR list [e, e1): lane l holds entry base + l (clamped to
// e1 - 1), refilled when e leaves the window.  The clamp ties the window to one
// list: call reset() before reading another list.
// Two per-tile floats (scales) can ride along: gathered from sa[tile] and
// sb[tile] when the window is refilled, read back the same way, so that no
// scalar-memory load sits in the tile loop (its lgkmcnt would add to the
// hand-counted LDS waits).
struct EntryCache {
  int tile = 0, mask = 0, base = -(1 << 30);
  float s0 = 1.f, s1 = 1.f;
  __device__ __forceinline__ void reset() { base = -(1 << 30); }
  __device__ __forceinline__ void get(const int* ent, int e, int e1, int lane, int& t, int& m) {
    if (e - base >= 64 || e < base) {  // wave-uniform
      base = e;
      const int idx = min(e + lane, e1 - 1);
      tile = ent[2 * idx];
      mask = ent[2 * idx + 1];
    }
    t = __builtin_amdgcn_readlane(tile, e - base);
    m = __builtin_amdgcn_readlane(mask, e - base);
  }
  // also the row-entry index crow[e] of the entry (the dS slot under MATTN_BWD_DS)
  int rowi = 0;
  __device__ __forceinline__ void get(const int* ent, int e, int e1, int lane, int& t, int& m,
                                      const float* sa, const float* sb, float& a, float& b,
                                      const int* crow, int& ri) {
    if (e - base >= 64 || e < base) {  // wave-uniform
      base = e;
      const int idx = min(e + lane, e1 - 1);
      tile = ent[2 * idx];
      mask = ent[2 * idx + 1];
      rowi = crow[idx];
      s0 = sa[tile];
      s1 = sb[tile];
    }
    t = __builtin_amdgcn_readlane(tile, e - base);
    m = __builtin_amdgcn_readlane(mask, e - base);
    ri = __builtin_amdgcn_readlane(rowi, e - base);
    a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s0), e - base));
    b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s1), e - base));
  }
  __device__ __forceinline__ void get(const int* ent, int e, int e1, int lane, int& t, int& m,
                                      const float* sa, const float* sb, float& a, float& b) {
    if (e - base >= 64 || e < base) {  // wave-uniform
      base = e;
      const int idx = min(e + lane, e1 - 1);
      tile = ent[2 * idx];
      mask = ent[2 * idx + 1];
      s0 = sa[tile];
      s1 = sb[tile];
    }
    t = __builtin_amdgcn_readlane(tile, e - base);
    m = __builtin_amdgcn_readlane(mask, e - base);
    a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s0), e - base));
    b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s1), e - base));
  }
};

// Output rows of one wave from the MFMA C layout to global memory along the
// rows.  The wave holds 32 rows x D columns as acc[mt][4 j + i] = column
// 32 mt + 8 j + 4 hi + i of row l32 (scaled by sc on the way out); they are
// staged in `lds` (32 * D * ES bytes, this wave's alone) as rows of 16-byte
// chunks, chunk c of row r at c ^ (r % chunks-per-row), then read back so that
// each global store instruction writes whole rows, 16 bytes per lane.  Row r
// goes to out + ES * (row0 + r * rstride) when r < nrows.  ES = 4 stores
// float32, ES = 2 the 16-bit values pack2 makes.  NT: nontemporal stores
// (rows that no kernel of the step reads back soon).
// Rows whose bit in rmask is clear are not stored.
template <int D, int ES, bool NT, class Pack>
__device__ __forceinline__ void store_rows(const f32x16 (&acc)[D / 32], float sc, void* lds, void* out,
                                           int64_t row0, int64_t rstride, int nrows, int lane, Pack pack2,
                                           uint32_t rmask = 0xffffffffu) {
  constexpr int RB = D * ES;     // bytes per row
  constexpr int CPR = RB / 16;   // 16-byte chunks per row
  const int r = lane & 31, hi = lane >> 5;
  char* L = (char*)lds;
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * mt + 8 * j + 4 * hi;
      const float o0 = acc[mt][4 * j] * sc, o1 = acc[mt][4 * j + 1] * sc;
      const float o2 = acc[mt][4 * j + 2] * sc, o3 = acc[mt][4 * j + 3] * sc;
      if constexpr (ES == 4) {
        *(f32x4*)(L + r * RB + (((d >> 2) ^ (r & (CPR - 1))) << 4)) = f32x4{o0, o1, o2, o3};
      } else {
        *(u32x2*)(L + r * RB + (((d >> 3) ^ (r & (CPR - 1))) << 4) + 8 * hi) = u32x2{pack2(o0, o1), pack2(o2, o3)};
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 32 * CPR / 64; ++i) {
    const int n = 64 * i + lane;
    const int row = n / CPR, c = n % CPR;
    const u32x4 v = *(const u32x4*)(L + row * RB + ((c ^ (row & (CPR - 1))) << 4));
    u32x4* dst = (u32x4*)((char*)out + (int64_t)ES * (row0 + (int64_t)row * rstride) + 16 * c);
    if (row < nrows && ((rmask >> row) & 1u)) {
      if constexpr (NT) __builtin_nontemporal_store(v, dst);
      else *dst = v;
    }
  }
}

// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16-byte LDS read issued where it stands (asm volatile keeps its order
// against the other asm statements): hand-pipelined operand reads.  The
// compiler does not count it in its own lgkmcnt waits (those stay correct: LDS
// returns in order, so extra outstanding reads only lengthen them); the value
// may be used only after an lgkm_wait that covers it, passed through hold().
template <int OFF>
__device__ __forceinline__ u32x4 ds_read128(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
// Transposed 8-byte LDS read (ds_read_b64_tr_b16, lane mapping as at tr_src)
// issued where it stands, like ds_read128.
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr8(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
// s_waitcnt lgkmcnt(N) in the asm order; values read by ds_read128 /
// ds_read_tr8 before it are passed through hold() after it, so that nothing
// using them is scheduled ahead of the wait.  hold() also pins an MFMA result
// between two asm statements (the MFMA is then issued where it stands).
// s_waitcnt immediate that waits for at most n outstanding vector memory
// operations and leaves the other counters alone (gfx9 encoding)
constexpr int vmcnt_only(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }
template <int N>
__device__ __forceinline__ void lgkm_wait() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}
template <class T>
__device__ __forceinline__ void hold(T& x) {
  asm volatile("" : "+v"(x));
}

// x, re-defined by an empty asm: values computed from the result inside a loop
// are not hoisted out of it (trades a few VALU ops for registers held across the loop)
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ int map_row(const KArgs& a, int b, int h, int n, int t) {
  return ((a.map_b == 1 ? 0 : b) * a.map_h + (a.map_h == 1 ? 0 : h)) * n + t;
}

// One 128-row tile of a 16-bit [rows, D] tensor held by 512 threads, 4 per row
// (thread t: row t / 4, 16-byte chunks t % 4 + 4 j, j < CPL: the 4 threads of a
// row cover 64 contiguous bytes per access), and its conversion to float16
// times a power of two: tile_load, tile_absmax and block_max2_512 for the
// tile's max |x|, then chunk_f16 per chunk.
template <int D>
struct TileRows {
  static constexpr int CPL = D / 32;  // 16-byte chunks per thread
  u32x4 x[CPL];
  // chunk index within the row of this thread's chunk j
  static __device__ __forceinline__ int chunk(int part, int j) { return part + 4 * j; }
};

// Rows r >= n are zero.  src points at row 0; rs is the row stride in elements.
template <int D>
__device__ __forceinline__ void tile_load(TileRows<D>& t, const uint16_t* src, int64_t rs, int n) {
  const int r = threadIdx.x >> 2, part = threadIdx.x & 3;
#pragma unroll
  for (int j = 0; j < TileRows<D>::CPL; ++j) t.x[j] = u32x4{0u, 0u, 0u, 0u};
  if (r < n) {
    const uint16_t* p = src + (int64_t)r * rs;
#pragma unroll
    for (int j = 0; j < TileRows<D>::CPL; ++j) t.x[j] = *(const u32x4*)(p + 8 * TileRows<D>::chunk(part, j));
  }
}

// max |x| over this thread's values of a tile
template <int D, class Tag>
__device__ __forceinline__ float tile_absmax(const TileRows<D>& t) {
  using E = Elt<Tag>;
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < TileRows<D>::CPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(E::to_f32(elt16(t.x[j], e))));
  return m;
}

// Workgroup barrier that waits for this wave's LDS operations (lgkmcnt(0))
// but not for its vector memory operations, unlike __syncthreads, whose fence
// also drains loads in flight (and stores); asm, so that the compiler moves no
// memory operation across it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// The same barrier where global->LDS loads may stay in flight on purpose (it
// hands no DMA-filled buffer to the other waves); the comment marks it for the
// assembly check of tests/lds_waits.py.
__device__ __forceinline__ void barrier_lds_dma_in_flight() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier ; lds-only: global->LDS loads may be in flight" ::: "memory");
}

// maximum over the 512 threads of a workgroup (red: 8 entries; one barrier
// before the write guards a previous use of red)
__device__ __forceinline__ f32x2 block_max2_512(f32x2 x, f32x2* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    x[0] = fmaxf(x[0], __shfl_xor(x[0], o));
    x[1] = fmaxf(x[1], __shfl_xor(x[1], o));
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  f32x2 r = red[0];
#pragma unroll
  for (int w = 1; w < 8; ++w) {
    r[0] = fmaxf(r[0], red[w][0]);
    r[1] = fmaxf(r[1], red[w][1]);
  }
  return r;
}

// float16 x * s of chunk j (s a power of two: exact for bfloat16 and float16
// values whose product stays in float16's range)
template <class Tag>
__device__ __forceinline__ u32x4 chunk_f16(const u32x4& x, float s) {
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  u32x4 y;
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = H::pack2(E::to_f32(elt16(x, 2 * e)) * s, E::to_f32(elt16(x, 2 * e + 1)) * s);
  return y;
}

}  // namespace mattn
