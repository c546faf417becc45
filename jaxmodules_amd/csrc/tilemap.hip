// Device tile-map classifier: the tile classification of create_block_mask
// (/root/reference/jaxmodules/block_mask.py:454-498, get_partial_block
// :381-408) and of the host tracer, done on the GPU for masks given in closed
// form (causal, element window, document ids, a per-tile table, keys in the
// query's residue class modulo a period, and the reference's visited-key-block
// window, attention.py:161-167,199-204).
//
// One wave per 128 x 128 tile.  Lane l owns query rows l and l + 64 of the
// tile and builds their key bitmasks (two 64-bit words each, the row_bits
// layout of mattn_blockmap).  Every predicate except document equality and
// the residue class is an interval of keys per query row, so a row's words
// come from two shifts; the residue class keeps every P-th key of the row from
// its first one in the tile; the
// document predicate is applied row by row with a ballot over the tile's
// keys, and only in tiles whose document ids neither all agree nor are
// disjoint.  The classifier writes per tile its state (absent / full /
// partial), its allowed-element count and a 128-bit hash of a partial tile's
// bits; the host de-duplicates partial tiles by hash and assembles the lists,
// and mattn_tilemap_bits writes (and verifies) the distinct masks.
#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

#include "mattn.h"

namespace mattn {
namespace {

constexpr int TILE = 128;

struct TMArgs {
  int causal, wl, wr;
  int doc_b;
  const int32_t* doc_q;
  const int32_t* doc_k;
  int tab_b, tab_h;
  const uint8_t* tiles;
  int bs, lwb, rwb, bnk;
  int Lq, Lk, map_b, map_h, nqt, nkt;
  int period;  // > 1: keys with (q - k) % period == 0 only
};

// keys [a, e) of a 64-key word (a and e relative to the word's first key)
__device__ __forceinline__ uint64_t span_bits(int a, int e) {
  a = max(a, 0);
  e = min(e, 64);
  if (e <= a) return 0;
  const uint64_t hi = e == 64 ? ~0ull : ((1ull << e) - 1);
  return hi & (~0ull << a);
}

// [lo, hi) of the keys allowed for query q by every predicate except document
// equality; tv is the tile table entry (1: only the range and visited blocks)
__device__ __forceinline__ void row_span(const TMArgs& a, int q, int tv, int& lo, int& hi) {
  lo = 0;
  hi = a.Lk;
  if (q >= a.Lq) {
    hi = 0;
    return;
  }
  if (tv == 2) {
    if (a.causal) hi = min(hi, q + 1);
    if (a.wl >= 0) lo = (int)max((long long)lo, (long long)q - a.wl);
    if (a.wr >= 0) hi = (int)min((long long)hi, (long long)q + a.wr + 1);
  }
  if (a.bs > 0) {
    const int w = a.lwb + a.rwb;
    int s = max(q / a.bs - a.lwb, 0);
    s = min(s, a.bnk - w);
    lo = (int)max((long long)lo, (long long)s * a.bs);
    hi = (int)min((long long)hi, (long long)(s + w) * a.bs);
  }
}

__device__ __forceinline__ int wave_min(int x) {
  for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ int wave_max(int x) {
  for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ uint64_t wave_sum64(uint64_t x) {
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)x, o), hi = __shfl_xor((uint32_t)(x >> 32), o);
    x += ((uint64_t)hi << 32) | lo;
  }
  return x;
}

// splitmix64 finaliser (Steele, Lea, Flood 2014), a bijective 64-bit mixer
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// The tile's row words: w[s][h] = keys 64h..64h+63 of query row lane + 64 s.
// Wave-uniform arguments; returns the table entry.
__device__ int tile_words(const TMArgs& a, int mb, int mh, int qt, int kt, int lane, uint64_t w[2][2]) {
  int tv = 2;
  if (a.tab_b > 0) {
    const int tb = a.tab_b == 1 ? 0 : mb, th = a.tab_h == 1 ? 0 : mh;
    tv = a.tiles[(((int64_t)tb * a.tab_h + th) * a.nqt + qt) * a.nkt + kt];
  }
  const int k0 = kt * TILE;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    int lo = 0, hi = 0;
    if (tv != 0) row_span(a, qt * TILE + lane + 64 * s, tv, lo, hi);
    w[s][0] = span_bits(lo - k0, hi - k0);
    w[s][1] = span_bits(lo - k0 - 64, hi - k0 - 64);
    if (a.period > 1 && tv == 2) {
      // keys k0 + j with j = (q - k0) mod period + m period
      const int q = qt * TILE + lane + 64 * s;
      const int j0 = ((q - k0) % a.period + a.period) % a.period;
      uint64_t r0 = 0, r1 = 0;
      for (int j = j0; j < TILE; j += a.period) {
        if (j < 64) r0 |= 1ull << j;
        else r1 |= 1ull << (j - 64);
      }
      w[s][0] &= r0;
      w[s][1] &= r1;
    }
  }
  if (a.doc_b > 0 && tv == 2 && __ballot((w[0][0] | w[0][1] | w[1][0] | w[1][1]) != 0) != 0) {
    const int bd = a.doc_b == 1 ? 0 : mb;
    const int32_t* dq = a.doc_q + (int64_t)bd * a.Lq;
    const int32_t* dk = a.doc_k + (int64_t)bd * a.Lk;
    const int qa = qt * TILE + lane, qb = qa + 64, ka = k0 + lane, kb = ka + 64;
    const int dqa = dq[min(qa, a.Lq - 1)], dqb = dq[min(qb, a.Lq - 1)];
    const int dka = dk[min(ka, a.Lk - 1)], dkb = dk[min(kb, a.Lk - 1)];
    // ranges over the rows and keys in bounds (the others have empty words)
    const int qmin = wave_min(min(qa < a.Lq ? dqa : INT_MAX, qb < a.Lq ? dqb : INT_MAX));
    const int qmax = wave_max(max(qa < a.Lq ? dqa : INT_MIN, qb < a.Lq ? dqb : INT_MIN));
    const int kmin = wave_min(min(ka < a.Lk ? dka : INT_MAX, kb < a.Lk ? dkb : INT_MAX));
    const int kmax = wave_max(max(ka < a.Lk ? dka : INT_MIN, kb < a.Lk ? dkb : INT_MIN));
    if (qmax < kmin || qmin > kmax) {
      w[0][0] = w[0][1] = w[1][0] = w[1][1] = 0;      // no common document
    } else if (!(qmin == qmax && kmin == kmax)) {     // else: one document for all
      for (int r = 0; r < 64; ++r) {
        const int d0 = __builtin_amdgcn_readlane(dqa, r), d1 = __builtin_amdgcn_readlane(dqb, r);
        const uint64_t m00 = __ballot(dka == d0), m01 = __ballot(dkb == d0);
        const uint64_t m10 = __ballot(dka == d1), m11 = __ballot(dkb == d1);
        if (lane == r) {
          w[0][0] &= m00;
          w[0][1] &= m01;
          w[1][0] &= m10;
          w[1][1] &= m11;
        }
      }
    }
  }
  return tv;
}

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void tilemap_classify(TMArgs a, int64_t ntiles, int8_t* state, int32_t* count, uint64_t* hash) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= ntiles) return;
  const int kt = (int)(t % a.nkt);
  const int64_t r = t / a.nkt;
  const int qt = (int)(r % a.nqt);
  const int m = (int)(r / a.nqt);
  const int mb = m / a.map_h, mh = m % a.map_h;
  uint64_t w[2][2];
  tile_words(a, mb, mh, qt, kt, lane, w);
  const bool any = __ballot((w[0][0] | w[0][1] | w[1][0] | w[1][1]) != 0) != 0;
  const bool all = __ballot((w[0][0] & w[0][1] & w[1][0] & w[1][1]) == ~0ull) == ~0ull;
  const uint64_t cnt = wave_sum64((uint64_t)(__popcll(w[0][0]) + __popcll(w[0][1]) +
                                             __popcll(w[1][0]) + __popcll(w[1][1])));
  const int st = !any ? 0 : all ? 1 : 2;
  uint64_t h1 = 0, h2 = 0;
  if (st == 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint64_t idx = (uint64_t)(h * TILE + lane + 64 * s);    // row_bits word index
        h1 += mix64(w[s][h] ^ (idx * 0x9e3779b97f4a7c15ull));
        h2 += mix64(w[s][h] + mix64(idx + 0x632be59bd9b4e019ull));
      }
    h1 = wave_sum64(h1);
    h2 = wave_sum64(h2);
  }
  if (lane == 0) {
    state[t] = (int8_t)st;
    count[t] = (int32_t)cnt;
    hash[2 * t] = h1;
    hash[2 * t + 1] = h2;
  }
}

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void tilemap_bits(TMArgs a, int64_t ntiles, const int32_t* list, int n, int n_masks, int write,
                  uint64_t* row_bits, uint64_t* col_bits, int32_t* mismatch) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const int64_t t = list[2 * i];
  const int64_t mid = list[2 * i + 1];
  if (t < 0 || t >= ntiles || mid < 0 || mid >= n_masks) return;  // entries out of range are skipped
  const int kt = (int)(t % a.nkt);
  const int64_t r = t / a.nkt;
  const int qt = (int)(r % a.nqt);
  const int m = (int)(r / a.nqt);
  uint64_t w[2][2];
  tile_words(a, m / a.map_h, m % a.map_h, qt, kt, lane, w);
  uint64_t* rb = row_bits + mid * 2 * TILE;
  if (!write) {
    bool bad = false;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) bad |= rb[h * TILE + lane + 64 * s] != w[s][h];
    if (bad) *mismatch = 1;
    return;
  }
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) rb[h * TILE + lane + 64 * s] = w[s][h];
  // transpose: col word [hq][key] bit j = query row 64 hq + j allows the key;
  // lane owns keys lane (word half 0) and lane + 64 (half 1)
  uint64_t c[2][2] = {{0, 0}, {0, 0}};   // [hq][key half]
  for (int j = 0; j < 64; ++j) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)w[s][h], j);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(w[s][h] >> 32), j);
        const uint64_t row = ((uint64_t)hi << 32) | lo;
        c[s][h] |= ((row >> lane) & 1ull) << j;
      }
    }
  }
  uint64_t* cb = col_bits + mid * 2 * TILE;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) cb[s * TILE + lane + 64 * h] = c[s][h];
}

int check_spec(const mattn_maskspec* ms, int32_t Lq, int32_t Lk, int32_t map_b, int32_t map_h,
               TMArgs& a, int64_t& ntiles) {
  if (!ms) return MATTN_ERR_NULL;
  if (Lq <= 0 || Lk <= 0 || map_b <= 0 || map_h <= 0) return MATTN_ERR_SHAPE;
  const int64_t nqt = (Lq + TILE - 1) / TILE, nkt = (Lk + TILE - 1) / TILE;
  ntiles = (int64_t)map_b * map_h * nqt * nkt;
  if (ntiles >= INT32_MAX / 2) return MATTN_ERR_TOO_LARGE;
  if (ms->causal != 0 && ms->causal != 1) return MATTN_ERR_SHAPE;
  if (ms->win_left < -1 || ms->win_right < -1) return MATTN_ERR_SHAPE;
  if (ms->doc_b != 0 && ms->doc_b != 1 && ms->doc_b != map_b) return MATTN_ERR_SHAPE;
  if (ms->doc_b != 0 && (!ms->doc_q || !ms->doc_k)) return MATTN_ERR_NULL;
  if (ms->tab_b != 0) {
    if (ms->tab_b != 1 && ms->tab_b != map_b) return MATTN_ERR_SHAPE;
    if (ms->tab_h != 1 && ms->tab_h != map_h) return MATTN_ERR_SHAPE;
    if (!ms->tiles) return MATTN_ERR_NULL;
  }
  if (ms->blk_size < 0 || ms->res_period < 0) return MATTN_ERR_SHAPE;
  if (ms->blk_size > 0) {
    if (ms->blk_left < 0 || ms->blk_right < 0 || ms->blk_left + ms->blk_right <= 0 ||
        ms->blk_nk < ms->blk_left + ms->blk_right)
      return MATTN_ERR_SHAPE;
  }
  a = TMArgs{ms->causal, ms->win_left, ms->win_right, ms->doc_b, ms->doc_q, ms->doc_k,
             ms->tab_b, ms->tab_b ? ms->tab_h : 0, ms->tiles, ms->blk_size, ms->blk_left,
             ms->blk_right, ms->blk_nk, Lq, Lk, map_b, map_h, (int)nqt, (int)nkt, ms->res_period};
  return MATTN_OK;
}

}  // namespace
}  // namespace mattn

using namespace mattn;

extern "C" {

int mattn_maskspec_validate(const mattn_maskspec* ms, int32_t Lq, int32_t Lk, int32_t map_b,
                            int32_t map_h) {
  TMArgs a;
  int64_t nt;
  return check_spec(ms, Lq, Lk, map_b, map_h, a, nt);
}

int mattn_tilemap_classify(const mattn_maskspec* ms, int32_t Lq, int32_t Lk, int32_t map_b,
                           int32_t map_h, int8_t* state, int32_t* count, uint64_t* hash,
                           void* stream) {
  TMArgs a;
  int64_t nt;
  const int rc = check_spec(ms, Lq, Lk, map_b, map_h, a, nt);
  if (rc != MATTN_OK) return rc;
  if (!state || !count || !hash) return MATTN_ERR_NULL;
  const int64_t grid = (nt + 3) / 4;
  hipLaunchKernelGGL(tilemap_classify, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a,
                     nt, state, count, hash);
  return hipGetLastError() == hipSuccess ? MATTN_OK : MATTN_ERR_LAUNCH;
}

int mattn_tilemap_bits(const mattn_maskspec* ms, int32_t Lq, int32_t Lk, int32_t map_b,
                       int32_t map_h, const int32_t* list, int32_t n, int32_t n_masks,
                       int32_t write, uint64_t* row_bits, uint64_t* col_bits, int32_t* mismatch,
                       void* stream) {
  TMArgs a;
  int64_t nt;
  const int rc = check_spec(ms, Lq, Lk, map_b, map_h, a, nt);
  if (rc != MATTN_OK) return rc;
  if (n < 0 || n_masks < 0) return MATTN_ERR_SHAPE;
  if (n == 0) return MATTN_OK;
  if (!list || !row_bits || (write && !col_bits) || (!write && !mismatch)) return MATTN_ERR_NULL;
  hipLaunchKernelGGL(tilemap_bits, dim3((unsigned)((n + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, a, nt, list, n, n_masks, write, row_bits, col_bits, mismatch);
  return hipGetLastError() == hipSuccess ? MATTN_OK : MATTN_ERR_LAUNCH;
}

}  // extern "C"
