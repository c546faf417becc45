// Backward pass of the masked attention (the custom_vjp bwd rule,
// /root/reference/jaxmodules/attention.py:266-342).
//
// The reference recomputes each query block's key scan and back-propagates
// through it, adding full-size dK/dV contributions per query block.  Here the
// gradient is computed from the saved base-2 log-sum-exp in three kernels:
//   bwd_pre  : delta = rowsum(dO * O) per query row; dO converted to the MFMA
//              dtype when O is float32;
//   bwd_dkdv : one workgroup per 128-key map column of (b, kv head); it walks
//              the column's present query tiles for every query head of the
//              GQA group and accumulates dK, dV in registers -- each element
//              written exactly once, no atomics;
//   bwd_dq   : one workgroup per 128-query map row; dQ accumulated in registers.
// With P = exp2(scale_log2 * S - lse) and dS = P * (dO V^T - delta):
//   dV = P^T dO,  dK = scale * dS^T Q,  dQ = scale * dS K.
#include "common.hpp"

namespace mattn {

// ---------------------------------------------------------------------------
// preprocess
// ---------------------------------------------------------------------------
// The dV product P^T dO runs on float16 MFMA: P lies in [0, 1] and float16
// keeps 11 significant bits against bfloat16's 8, which matters because dO
// arrives in float32 (the reference's output dtype).  dO is scaled by a power
// of two s so that max |dO * s| < 2^14 (the scale is exact and undone on the
// float32 result).  s comes from a deterministic two-pass max: bwd_absmax
// writes NPART partial maxima, bwd_pre reduces them.

// Element loads of one 16-lane row group: PER = D / 16 consecutive values.
template <int D, class Tag, bool O_F32>
__device__ __forceinline__ void load_row(const void* base, int64_t off, int sub, float* g) {
  using E = Elt<Tag>;
  constexpr int PER = D / 16;
  if constexpr (O_F32) {
    const float* p = (const float*)base + off + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4) {
      const f32x4 y = *(const f32x4*)(p + i);
      g[i] = y[0]; g[i + 1] = y[1]; g[i + 2] = y[2]; g[i + 3] = y[3];
    }
  } else {
    const uint16_t* p = (const uint16_t*)base + off + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4) {
      const u32x2 y = *(const u32x2*)(p + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) g[i + j] = E::to_f32((y[j >> 1] >> (16 * (j & 1))) & 0xffffu);
    }
  }
}

__device__ __forceinline__ float block_max256(float x, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// NPART workgroups; grid-stride over (b, q, h) rows, 16 lanes per row, four
// rows in flight per lane group.
template <int D, class Tag, bool O_F32>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void bwd_absmax(KArgs a) {
  constexpr int PER = D / 16;
  constexpr int UNR = 4;
  __shared__ float red[4];
  const uint32_t nrows = (uint32_t)a.B * a.Lq * a.Hq;  // < 2^31 (checked by the C ABI)
  const int sub = threadIdx.x & 15;
  const uint32_t step = gridDim.x * 16;
  float mx = 0.f;
  for (uint32_t r0 = blockIdx.x * 16 + (threadIdx.x >> 4); r0 < nrows; r0 += UNR * step) {
    float g[UNR][PER];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const uint32_t row = min(r0 + u * step, nrows - 1);  // a repeated row leaves the max unchanged
      const int h = (int)(row % (uint32_t)a.Hq);
      const uint32_t bq = row / (uint32_t)a.Hq;
      const int q = (int)(bq % (uint32_t)a.Lq), b = (int)(bq / (uint32_t)a.Lq);
      load_row<D, Tag, O_F32>(a.dO, (int64_t)b * a.dos[0] + (int64_t)q * a.dos[1] + (int64_t)h * a.dos[2],
                              sub, g[u]);
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u)
#pragma unroll
      for (int i = 0; i < PER; ++i) mx = fmaxf(mx, fabsf(g[u][i]));
  }
  mx = block_max256(mx, red);
  if (threadIdx.x == 0) a.part[blockIdx.x] = mx;
}

// One workgroup: the power-of-two scale s with max |dO * s| < 2^14, and 1/s.
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void bwd_scale(KArgs a) {
  __shared__ float red[4];
  float m = 0.f;
  for (int i = threadIdx.x; i < NPART; i += 256) m = fmaxf(m, a.part[i]);
  m = block_max256(m, red);
  if (threadIdx.x == 0) {
    float s = 1.f;
    if (m > 0.f && m <= 3.4e38f) {
      int e;
      frexpf(m, &e);  // m < 2^e
      s = ldexpf(1.f, min(126, max(-126, 14 - e)));
    }
    a.dscale[0] = s;
    a.dscale[1] = 1.f / s;
  }
}

// 16 lanes per (b, q, h) row, 16 rows per workgroup.  MODE 0: delta only
// (float32 inputs); 1: also dO * s in float16 (float16 inputs); 2: also dO in
// bfloat16 (bfloat16 inputs).
template <int D, class Tag, bool O_F32, int MODE>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void bwd_pre(KArgs a) {
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  constexpr int PER = D / 16;
  const uint32_t nrows = (uint32_t)a.B * a.Lq * a.Hq;  // < 2^31 (checked by the C ABI)
  const uint32_t row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (row >= nrows) return;  // uniform per 16-lane group; no barrier below
  const float s = MODE > 0 ? a.dscale[0] : 1.f;
  const int h = (int)(row % (uint32_t)a.Hq);
  const uint32_t bq = row / (uint32_t)a.Hq;
  const int q = (int)(bq % (uint32_t)a.Lq), b = (int)(bq / (uint32_t)a.Lq);
  float x[PER], g[PER];
  load_row<D, Tag, O_F32>(a.o, (int64_t)b * a.os[0] + (int64_t)q * a.os[1] + (int64_t)h * a.os[2], sub, x);
  load_row<D, Tag, O_F32>(a.dO, (int64_t)b * a.dos[0] + (int64_t)q * a.dos[1] + (int64_t)h * a.dos[2],
                          sub, g);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) acc = fmaf(x[i], g[i], acc);
  acc += __shfl_xor(acc, 1, 16);
  acc += __shfl_xor(acc, 2, 16);
  acc += __shfl_xor(acc, 4, 16);
  acc += __shfl_xor(acc, 8, 16);
  if (sub == 0) a.delta[((int64_t)b * a.Hq + h) * a.Lq + q] = acc;
  if constexpr (MODE > 0) {
    // dense [B, Lq, Hq, D] copies
    uint16_t* w = (uint16_t*)a.dOhw + (int64_t)row * D + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4)
      *(u32x2*)(w + i) = u32x2{H::pack2(g[i] * s, g[i + 1] * s), H::pack2(g[i + 2] * s, g[i + 3] * s)};
  }
  if constexpr (MODE == 2) {
    uint16_t* w = (uint16_t*)a.dO16w + (int64_t)row * D + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4)
      *(u32x2*)(w + i) = u32x2{E::pack2(g[i], g[i + 1]), E::pack2(g[i + 2], g[i + 3])};
  }
}

// ---------------------------------------------------------------------------
// dQ (MFMA)
// ---------------------------------------------------------------------------
// Each wave owns 32 queries; per 64-key sub-block:
//   S^T  = K Q^T         (A: K rows from LDS, B: Q^T in registers)
//   dP^T = V dO^T        (A: V rows from LDS, B: dO^T in registers)
//   dS^T = P^T * (dP^T - delta)    (each lane owns one query: lse, delta scalars)
//   dQ^T += K^T dS^T     (A: K^T by transposed reads of the same K tile)
// K and V are double-buffered, swizzled row-major tiles filled by direct
// global->LDS loads.
template <int D, class Tag>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bwd_dq_mfma(KArgs a) {
  using E = Elt<Tag>;
  using TL = TileLoad<D>;
  constexpr bool IS_BF16 = __is_same(Tag, bf16_tag);
  constexpr int BN = 64;
  constexpr int NKD = D / 16;
  constexpr int NMD = D / 32;
  constexpr int NI = D / 32;       // load instructions per wave per tile
  constexpr int BLK = 512;         // elements one load instruction fills

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][BN * D];

  const int item = a.q_order[blockIdx.x];
  if (item < 0) return;
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  const int nsb = 2 * (e1 - e0);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int qloc = wave * 32 + l32;
  const int q = qt * TILE + qloc;
  const int qc = min(q, a.Lq - 1);
  const float c2 = a.scale_log2;

  u32x4 qf[NKD], df[NKD];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (int64_t)b * a.qs[0] + (int64_t)qc * a.qs[1] +
                         (int64_t)h * a.qs[2] + 8 * hi;
    // bfloat16 inputs: dO rounded to bfloat16; float16 inputs: dO * s in float16
    const void* dsrc = IS_BF16 ? a.dO16 : a.dOh;
    const uint16_t* dp = (const uint16_t*)dsrc + (((int64_t)b * a.Lq + qc) * a.Hq + h) * D + 8 * hi;
#pragma unroll
    for (int kd = 0; kd < NKD; ++kd) {
      qf[kd] = *(const u32x4*)(qp + 16 * kd);
      df[kd] = *(const u32x4*)(dp + 16 * kd);
    }
  }
  const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + qc;
  const float nlse = -a.lse[rs];
  const float dl = a.delta[rs];
  const float dps = IS_BF16 ? 1.f : a.dscale[1];  // undoes the dO scale of float16 inputs

  const uint16_t* kb = (const uint16_t*)a.k + (int64_t)b * a.ks[0] + (int64_t)hk * a.ks[2];
  const uint16_t* vb = (const uint16_t*)a.v + (int64_t)b * a.vs[0] + (int64_t)hk * a.vs[2];
  uint32_t kld[NI], vld[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    kld[i] = TL::src_off(NI * wave + i, lane, a.ks[1]);
    vld[i] = TL::src_off(NI * wave + i, lane, a.vs[1]);
  }
  int rro[NKD];               // row-read offsets (K and V tiles share the layout)
#pragma unroll
  for (int kd = 0; kd < NKD; ++kd) rro[kd] = sw_off<D>(l32, 2 * kd + hi);
  int kto[NMD][2];            // K^T transposed-read offsets
#pragma unroll
  for (int mt = 0; mt < NMD; ++mt) {
    kto[mt][0] = tr_src<D>(lane, mt, 0);
    kto[mt][1] = tr_src<D>(lane, mt, 1);
  }

  auto issue = [&](int s, int buf) {
    const int kt = a.row_ent[2 * (e0 + (s >> 1))];
    const int key0 = kt * TILE + (s & 1) * BN;
    uint16_t* kl = &Ks[buf][NI * wave * BLK];
    uint16_t* vl = &Vs[buf][NI * wave * BLK];
    if (key0 + BN <= a.Lk) {
      const uint16_t* kp = kb + (int64_t)key0 * a.ks[1];
      const uint16_t* vp = vb + (int64_t)key0 * a.vs[1];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        lds_load16(kp + kld[i], kl + i * BLK);
        lds_load16(vp + vld[i], vl + i * BLK);
      }
    } else {  // ragged last sub-block: rows past Lk re-read row Lk-1 (masked anyway)
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int key = min(key0 + TL::row_of(NI * wave + i, lane), a.Lk - 1);
        const int c = TL::chunk_of(NI * wave + i, lane);
        lds_load16(kb + (int64_t)key * a.ks[1] + 8 * c, kl + i * BLK);
        lds_load16(vb + (int64_t)key * a.vs[1] + 8 * c, vl + i * BLK);
      }
    }
  };

  f32x16 acc[NMD];
#pragma unroll
  for (int i = 0; i < NMD; ++i) acc[i] = f32x16{};

  auto step = [&](int buf, bool masked, uint64_t mw) {
    f32x16 st[2], dp[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      u32x4 ka[NKD], va[NKD];
#pragma unroll
      for (int kd = 0; kd < NKD; ++kd) {
        ka[kd] = *(const u32x4*)&Ks[buf][rro[kd] + 32 * t * D];
        va[kd] = *(const u32x4*)&Vs[buf][rro[kd] + 32 * t * D];
      }
      st[t] = f32x16{};
      dp[t] = f32x16{};
#pragma unroll
      for (int kd = 0; kd < NKD; ++kd) {
        st[t] = E::mfma(ka[kd], qf[kd], st[t]);
        dp[t] = E::mfma(va[kd], df[kd], dp[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) st[t][r] = fast_exp2(fmaf(st[t][r], c2, nlse));
    if (masked) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t w32 = (uint32_t)(mw >> (32 * t)) >> (4 * hi);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!mask_bit(w32, r)) st[t][r] = 0.f;
      }
    }
    u32x4 pk[4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float d0 = st[t][r] * fmaf(dp[t][r], dps, -dl);
        const float d1 = st[t][r + 1] * fmaf(dp[t][r + 1], dps, -dl);
        pk[2 * t + (r >> 3)][(r & 7) >> 1] = E::pack2(d0, d1);
      }
    }
#pragma unroll
    for (int mt = 0; mt < NMD; ++mt) {
      u32x4 ta[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x2 lo = lds_read_tr(&Ks[buf][kto[mt][0] + 16 * ks * D]);
        const u32x2 up = lds_read_tr(&Ks[buf][kto[mt][1] + 16 * ks * D]);
        ta[ks] = u32x4{lo[0], lo[1], up[0], up[1]};
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc[mt] = E::mfma(ta[ks], pk[ks], acc[mt]);
    }
  };

  if (nsb > 0) issue(0, 0);
  for (int s = 0; s < nsb; ++s) {
    const int buf = s & 1;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int mask = a.row_ent[2 * (e0 + (s >> 1)) + 1];
    uint64_t mw = 0;
    if (mask >= 0) mw = a.row_bits[((int64_t)mask * TILE + qloc) * 2 + (s & 1)];
    if (s + 1 < nsb) issue(s + 1, buf ^ 1);
    step(buf, mask >= 0, mw);
  }

  if (q >= a.Lq) return;
  char* op = (char*)a.dq;
  const int64_t orow = (int64_t)b * a.dqs[0] + (int64_t)q * a.dqs[1] + (int64_t)h * a.dqs[2];
#pragma unroll
  for (int mt = 0; mt < NMD; ++mt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * mt + 8 * j + 4 * hi;
      *(u32x2*)(op + 2 * (orow + d)) =
          u32x2{E::pack2(acc[mt][4 * j] * a.scale, acc[mt][4 * j + 1] * a.scale),
                E::pack2(acc[mt][4 * j + 2] * a.scale, acc[mt][4 * j + 3] * a.scale)};
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV (MFMA, no atomics)
// ---------------------------------------------------------------------------
// Each wave owns 32 keys; per 64-query sub-block:
//   S    = Q K^T          (A: Q rows from LDS, B: K^T in registers)
//   dP   = dO V^T         (A: dO rows from LDS, B: V^T in registers)
//   P    = exp2(scale_log2 S - lse),  dS = P * (dP - delta)
//   dV^T += dO^T P        (A: transposed reads of the float16 dO * s tile;
//                          float16 MFMA)
//   dK^T += Q^T dS        (A: transposed reads of the Q tile)
// Q, dO (and, for bfloat16 inputs, the separate float16 dO * s tile), lse and
// delta are double-buffered in LDS and filled by direct global->LDS loads.
template <int D, class Tag>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bwd_dkdv_mfma(KArgs a) {
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  using TL = TileLoad<D>;
  constexpr bool IS_BF16 = __is_same(Tag, bf16_tag);
  constexpr int BM = 64;           // queries per sub-block
  constexpr int NKD = D / 16;
  constexpr int NMD = D / 32;
  constexpr int NI = D / 32;
  constexpr int BLK = 512;
  constexpr int NH = IS_BF16 ? 2 : 1;  // float16 dO * s tile: separate (bf16) or the dO tile

  __shared__ __attribute__((aligned(16))) uint16_t Qs[2][BM * D];
  __shared__ __attribute__((aligned(16))) uint16_t Ds[2][BM * D];
  __shared__ __attribute__((aligned(16))) uint16_t Hs[NH == 2 ? 2 : 1][NH == 2 ? BM * D : 8];
  __shared__ __attribute__((aligned(16))) float Ls[2][BM];
  __shared__ __attribute__((aligned(16))) float Dl[2][BM];

  const int item = a.kv_order[blockIdx.x];
  if (item < 0) return;
  const int kt = item % a.nkt;
  const int bh = item / a.nkt;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int kloc = wave * 32 + l32;
  const int key = kt * TILE + kloc;
  const int kcl = min(key, a.Lk - 1);
  const float c2 = a.scale_log2;

  u32x4 kf[NKD], vf[NKD];
  {
    const uint16_t* kp = (const uint16_t*)a.k + (int64_t)b * a.ks[0] + (int64_t)kcl * a.ks[1] +
                         (int64_t)hk * a.ks[2] + 8 * hi;
    const uint16_t* vp = (const uint16_t*)a.v + (int64_t)b * a.vs[0] + (int64_t)kcl * a.vs[1] +
                         (int64_t)hk * a.vs[2] + 8 * hi;
#pragma unroll
    for (int kd = 0; kd < NKD; ++kd) {
      kf[kd] = *(const u32x4*)(kp + 16 * kd);
      vf[kd] = *(const u32x4*)(vp + 16 * kd);
    }
  }

  // Flattened walk over (query head g of the group, column entry, half).
  int tot = 0;
  for (int g = 0; g < a.G; ++g) {
    const int mc = map_row(a, b, hk * a.G + g, a.nkt, kt);
    tot += 2 * (a.col_ptr[mc + 1] - a.col_ptr[mc]);
  }
  // cursor of the next sub-block to load
  int lg = 0, le = 0, lend = 0, lhalf = 0;
  {
    const int mc = map_row(a, b, hk * a.G, a.nkt, kt);
    le = a.col_ptr[mc];
    lend = a.col_ptr[mc + 1];
  }

  const int64_t drow = (int64_t)a.Hq * D;   // row stride of the dense dO copies
  uint32_t qld[NI], dld[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    qld[i] = TL::src_off(NI * wave + i, lane, a.qs[1]);
    dld[i] = TL::src_off(NI * wave + i, lane, drow);
  }
  int rro[NKD];
#pragma unroll
  for (int kd = 0; kd < NKD; ++kd) rro[kd] = sw_off<D>(l32, 2 * kd + hi);
  int tro[NMD][2];
#pragma unroll
  for (int mt = 0; mt < NMD; ++mt) {
    tro[mt][0] = tr_src<D>(lane, mt, 0);
    tro[mt][1] = tr_src<D>(lane, mt, 1);
  }
  const float inv_s = a.dscale[1];
  const float dps = IS_BF16 ? 1.f : inv_s;
  int cmask_e = 0, chalf = 0;  // entry and half of the most recently issued sub-block

  auto issue = [&](int buf) {  // global -> LDS loads of the sub-block at the cursor
    while (le >= lend) {
      ++lg;
      const int mc = map_row(a, b, hk * a.G + lg, a.nkt, kt);
      le = a.col_ptr[mc];
      lend = a.col_ptr[mc + 1];
    }
    const int h = hk * a.G + lg;
    const int q0 = a.col_ent[2 * le] * TILE + lhalf * BM;
    const uint16_t* qb = (const uint16_t*)a.q + (int64_t)b * a.qs[0] + (int64_t)h * a.qs[2];
    const int64_t dro = ((int64_t)b * a.Lq * a.Hq + h) * D;
    const uint16_t* db = (const uint16_t*)(IS_BF16 ? a.dO16 : a.dOh) + dro;
    const uint16_t* hb = (const uint16_t*)a.dOh + dro;
    uint16_t* ql = &Qs[buf][NI * wave * BLK];
    uint16_t* dl_ = &Ds[buf][NI * wave * BLK];
    uint16_t* hl = &Hs[NH == 2 ? buf : 0][NH == 2 ? NI * wave * BLK : 0];
    if (q0 + BM <= a.Lq) {
      const uint16_t* qp = qb + (int64_t)q0 * a.qs[1];
      const uint16_t* dp = db + (int64_t)q0 * drow;
      const uint16_t* hp = hb + (int64_t)q0 * drow;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        lds_load16(qp + qld[i], ql + i * BLK);
        lds_load16(dp + dld[i], dl_ + i * BLK);
        if constexpr (NH == 2) lds_load16(hp + dld[i], hl + i * BLK);
      }
    } else {  // ragged last sub-block: rows past Lq re-read row Lq-1 (masked anyway)
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int qq = min(q0 + TL::row_of(NI * wave + i, lane), a.Lq - 1);
        const int c = TL::chunk_of(NI * wave + i, lane);
        lds_load16(qb + (int64_t)qq * a.qs[1] + 8 * c, ql + i * BLK);
        lds_load16(db + (int64_t)qq * drow + 8 * c, dl_ + i * BLK);
        if constexpr (NH == 2) lds_load16(hb + (int64_t)qq * drow + 8 * c, hl + i * BLK);
      }
    }
    if (wave < 2) {  // lse (wave 0) and delta (wave 1) of the 64 rows
      const int qq = min(q0 + lane, a.Lq - 1);
      const float* src = (wave == 0 ? a.lse : a.delta) + ((int64_t)b * a.Hq + h) * a.Lq + qq;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(wave == 0 ? Ls[buf] : Dl[buf]),
                                       4, 0, 0);
    }
    cmask_e = le;
    chalf = lhalf;
    if (lhalf == 0) {
      lhalf = 1;
    } else {
      lhalf = 0;
      ++le;
    }
  };

  f32x16 dk[NMD], dv[NMD];
#pragma unroll
  for (int i = 0; i < NMD; ++i) { dk[i] = f32x16{}; dv[i] = f32x16{}; }

  auto step = [&](int buf, bool masked, uint64_t mw) {
    const uint16_t* ht = NH == 2 ? Hs[buf] : Ds[buf];  // float16 dO * s tile
    f32x16 st[2], dp[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      u32x4 qa[NKD], da[NKD];
#pragma unroll
      for (int kd = 0; kd < NKD; ++kd) {
        qa[kd] = *(const u32x4*)&Qs[buf][rro[kd] + 32 * t * D];
        da[kd] = *(const u32x4*)&Ds[buf][rro[kd] + 32 * t * D];
      }
      st[t] = f32x16{};
      dp[t] = f32x16{};
#pragma unroll
      for (int kd = 0; kd < NKD; ++kd) {
        st[t] = E::mfma(qa[kd], kf[kd], st[t]);
        dp[t] = E::mfma(da[kd], vf[kd], dp[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 lv = *(const f32x4*)&Ls[buf][32 * t + 8 * j + 4 * hi];
#pragma unroll
        for (int i = 0; i < 4; ++i) st[t][4 * j + i] = fast_exp2(fmaf(st[t][4 * j + i], c2, -lv[i]));
      }
    }
    if (masked) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t w32 = (uint32_t)(mw >> (32 * t)) >> (4 * hi);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!mask_bit(w32, r)) st[t][r] = 0.f;
      }
    }
    u32x4 pk[4], sk[4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 dv4 = *(const f32x4*)&Dl[buf][32 * t + 8 * j + 4 * hi];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * j + i;
          dp[t][r] = st[t][r] * fmaf(dp[t][r], dps, -dv4[i]);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        pk[2 * t + (r >> 3)][(r & 7) >> 1] = H::pack2(st[t][r], st[t][r + 1]);
        sk[2 * t + (r >> 3)][(r & 7) >> 1] = E::pack2(dp[t][r], dp[t][r + 1]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < NMD; ++mt) {
      u32x4 ta[4], tb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x2 h0 = lds_read_tr(&ht[tro[mt][0] + 16 * ks * D]);
        const u32x2 h1 = lds_read_tr(&ht[tro[mt][1] + 16 * ks * D]);
        const u32x2 q0 = lds_read_tr(&Qs[buf][tro[mt][0] + 16 * ks * D]);
        const u32x2 q1 = lds_read_tr(&Qs[buf][tro[mt][1] + 16 * ks * D]);
        ta[ks] = u32x4{h0[0], h0[1], h1[0], h1[1]};
        tb[ks] = u32x4{q0[0], q0[1], q1[0], q1[1]};
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        dv[mt] = H::mfma(ta[ks], pk[ks], dv[mt]);
        dk[mt] = E::mfma(tb[ks], sk[ks], dk[mt]);
      }
    }
  };

  if (tot > 0) issue(0);
  for (int s = 0; s < tot; ++s) {
    const int buf = s & 1;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int mask = a.col_ent[2 * cmask_e + 1];
    const int half = chalf;
    uint64_t mw = 0;
    if (mask >= 0) mw = a.col_bits[((int64_t)mask * TILE + kloc) * 2 + half];
    if (s + 1 < tot) issue(buf ^ 1);
    step(buf, mask >= 0, mw);
  }

  if (key >= a.Lk) return;
  char* kp = (char*)a.dk;
  char* vp = (char*)a.dv;
  const int64_t krow = (int64_t)b * a.dks[0] + (int64_t)key * a.dks[1] + (int64_t)hk * a.dks[2];
  const int64_t vrow = (int64_t)b * a.dvs[0] + (int64_t)key * a.dvs[1] + (int64_t)hk * a.dvs[2];
#pragma unroll
  for (int mt = 0; mt < NMD; ++mt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * mt + 8 * j + 4 * hi;
      *(u32x2*)(kp + 2 * (krow + d)) =
          u32x2{E::pack2(dk[mt][4 * j] * a.scale, dk[mt][4 * j + 1] * a.scale),
                E::pack2(dk[mt][4 * j + 2] * a.scale, dk[mt][4 * j + 3] * a.scale)};
      *(u32x2*)(vp + 2 * (vrow + d)) =
          u32x2{E::pack2(dv[mt][4 * j] * inv_s, dv[mt][4 * j + 1] * inv_s),
                E::pack2(dv[mt][4 * j + 2] * inv_s, dv[mt][4 * j + 3] * inv_s)};
    }
  }
}

// ---------------------------------------------------------------------------
// float32 SIMT backward
// ---------------------------------------------------------------------------

template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void bwd_dq_simt(KArgs a) {
  constexpr int SB = 32;
  constexpr int DP = D / 4;
  __shared__ __attribute__((aligned(16))) float Ks[SB * D];
  __shared__ __attribute__((aligned(16))) float Vs[SB * D];

  const int item = a.q_order[blockIdx.x];
  if (item < 0) return;
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  const int tid = threadIdx.x, row = tid >> 2, part = tid & 3;
  const int q = qt * TILE + row;
  const int qc = min(q, a.Lq - 1);

  float qv[DP], gv[DP], dq[DP];
  {
    const float* qp = (const float*)a.q + (int64_t)b * a.qs[0] + (int64_t)qc * a.qs[1] +
                      (int64_t)h * a.qs[2] + part * DP;
    const float* gp = (const float*)a.dO + (int64_t)b * a.dos[0] + (int64_t)qc * a.dos[1] +
                      (int64_t)h * a.dos[2] + part * DP;
#pragma unroll
    for (int i = 0; i < DP; ++i) { qv[i] = qp[i]; gv[i] = gp[i]; dq[i] = 0.f; }
  }
  const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + qc;
  const float lse = a.lse[rs], dl = a.delta[rs];
  const float* kb = (const float*)a.k + (int64_t)b * a.ks[0] + (int64_t)hk * a.ks[2];
  const float* vb = (const float*)a.v + (int64_t)b * a.vs[0] + (int64_t)hk * a.vs[2];

  for (int e = e0; e < e1; ++e) {
    const int kt = a.row_ent[2 * e], mask = a.row_ent[2 * e + 1];
    for (int sb = 0; sb < TILE / SB; ++sb) {
      const int key0 = kt * TILE + sb * SB;
      if (key0 >= a.Lk) break;
      __syncthreads();
      for (int c = tid; c < SB * D / 4; c += 512) {
        const int r = c / (D / 4), col = 4 * (c % (D / 4));
        const int key = min(key0 + r, a.Lk - 1);
        *(f32x4*)&Ks[r * D + col] = *(const f32x4*)(kb + (int64_t)key * a.ks[1] + col);
        *(f32x4*)&Vs[r * D + col] = *(const f32x4*)(vb + (int64_t)key * a.vs[1] + col);
      }
      __syncthreads();
      uint32_t bits = 0xffffffffu;
      if (mask >= 0)
        bits = (uint32_t)(a.row_bits[((int64_t)mask * TILE + row) * 2 + (sb >> 1)] >> (32 * (sb & 1)));
      for (int j = 0; j < SB; ++j) {
        float s = 0.f, g = 0.f;
#pragma unroll
        for (int i = 0; i < DP; ++i) {
          s = fmaf(qv[i], Ks[j * D + part * DP + i], s);
          g = fmaf(gv[i], Vs[j * D + part * DP + i], g);
        }
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        g += __shfl_xor(g, 1);
        g += __shfl_xor(g, 2);
        float p = exp2f(s * a.scale_log2 - lse);
        if (!((bits >> j) & 1u)) p = 0.f;
        const float ds = p * (g - dl);
#pragma unroll
        for (int i = 0; i < DP; ++i) dq[i] = fmaf(ds, Ks[j * D + part * DP + i], dq[i]);
      }
    }
  }
  if (q >= a.Lq) return;
  float* op = (float*)a.dq + (int64_t)b * a.dqs[0] + (int64_t)q * a.dqs[1] + (int64_t)h * a.dqs[2] +
              part * DP;
#pragma unroll
  for (int i = 0; i < DP; ++i) op[i] = dq[i] * a.scale;
}

template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void bwd_dkdv_simt(KArgs a) {
  constexpr int SB = 32;
  constexpr int DP = D / 4;
  __shared__ __attribute__((aligned(16))) float Qs[SB * D];
  __shared__ __attribute__((aligned(16))) float Gs[SB * D];
  __shared__ float Ls[SB], Dl[SB];

  const int item = a.kv_order[blockIdx.x];
  if (item < 0) return;
  const int kt = item % a.nkt;
  const int bh = item / a.nkt;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  const int tid = threadIdx.x, row = tid >> 2, part = tid & 3;
  const int key = kt * TILE + row;
  const int kcl = min(key, a.Lk - 1);

  float kv[DP], vv[DP], dk[DP], dv[DP];
  {
    const float* kp = (const float*)a.k + (int64_t)b * a.ks[0] + (int64_t)kcl * a.ks[1] +
                      (int64_t)hk * a.ks[2] + part * DP;
    const float* vp = (const float*)a.v + (int64_t)b * a.vs[0] + (int64_t)kcl * a.vs[1] +
                      (int64_t)hk * a.vs[2] + part * DP;
#pragma unroll
    for (int i = 0; i < DP; ++i) { kv[i] = kp[i]; vv[i] = vp[i]; dk[i] = 0.f; dv[i] = 0.f; }
  }
  for (int g = 0; g < a.G; ++g) {
    const int h = hk * a.G + g;
    const int mc = map_row(a, b, h, a.nkt, kt);
    const int e0 = a.col_ptr[mc], e1 = a.col_ptr[mc + 1];
    const float* qb = (const float*)a.q + (int64_t)b * a.qs[0] + (int64_t)h * a.qs[2];
    const float* gb = (const float*)a.dO + (int64_t)b * a.dos[0] + (int64_t)h * a.dos[2];
    for (int e = e0; e < e1; ++e) {
      const int qt = a.col_ent[2 * e], mask = a.col_ent[2 * e + 1];
      for (int sb = 0; sb < TILE / SB; ++sb) {
        const int q0 = qt * TILE + sb * SB;
        if (q0 >= a.Lq) break;
        __syncthreads();
        for (int c = tid; c < SB * D / 4; c += 512) {
          const int r = c / (D / 4), col = 4 * (c % (D / 4));
          const int qq = min(q0 + r, a.Lq - 1);
          *(f32x4*)&Qs[r * D + col] = *(const f32x4*)(qb + (int64_t)qq * a.qs[1] + col);
          *(f32x4*)&Gs[r * D + col] = *(const f32x4*)(gb + (int64_t)qq * a.dos[1] + col);
        }
        if (tid < 2 * SB) {
          const int qq = min(q0 + (tid & (SB - 1)), a.Lq - 1);
          const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + qq;
          if (tid < SB) Ls[tid] = a.lse[rs];
          else Dl[tid - SB] = a.delta[rs];
        }
        __syncthreads();
        uint32_t bits = 0xffffffffu;
        if (mask >= 0)
          bits = (uint32_t)(a.col_bits[((int64_t)mask * TILE + row) * 2 + (sb >> 1)] >> (32 * (sb & 1)));
        for (int j = 0; j < SB; ++j) {
          float s = 0.f, gd = 0.f;
#pragma unroll
          for (int i = 0; i < DP; ++i) {
            s = fmaf(kv[i], Qs[j * D + part * DP + i], s);
            gd = fmaf(vv[i], Gs[j * D + part * DP + i], gd);
          }
          s += __shfl_xor(s, 1);
          s += __shfl_xor(s, 2);
          gd += __shfl_xor(gd, 1);
          gd += __shfl_xor(gd, 2);
          float p = exp2f(s * a.scale_log2 - Ls[j]);
          if (!((bits >> j) & 1u)) p = 0.f;
          const float ds = p * (gd - Dl[j]);
#pragma unroll
          for (int i = 0; i < DP; ++i) {
            dv[i] = fmaf(p, Gs[j * D + part * DP + i], dv[i]);
            dk[i] = fmaf(ds, Qs[j * D + part * DP + i], dk[i]);
          }
        }
      }
    }
  }
  if (key >= a.Lk) return;
  float* kp = (float*)a.dk + (int64_t)b * a.dks[0] + (int64_t)key * a.dks[1] + (int64_t)hk * a.dks[2] +
              part * DP;
  float* vp = (float*)a.dv + (int64_t)b * a.dvs[0] + (int64_t)key * a.dvs[1] + (int64_t)hk * a.dvs[2] +
              part * DP;
#pragma unroll
  for (int i = 0; i < DP; ++i) { kp[i] = dk[i] * a.scale; vp[i] = dv[i]; }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

hipError_t launch_bwd_stage(const KArgs& a, int D, int dtype, int o_dtype, int stage, int q_grid,
                            int kv_grid, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.Lq * a.Hq;
  const int pre_grid = (int)((rows + 15) / 16);
  const bool of32 = (o_dtype == MATTN_F32);
  if (dtype == MATTN_F32) {
    if (stage == MATTN_BWD_PRE) {
      if (D == 64) hipLaunchKernelGGL((bwd_pre<64, bf16_tag, true, 0>), dim3(pre_grid), dim3(256), 0, st, a);
      else hipLaunchKernelGGL((bwd_pre<128, bf16_tag, true, 0>), dim3(pre_grid), dim3(256), 0, st, a);
    } else if (stage == MATTN_BWD_DKDV) {
      if (D == 64) hipLaunchKernelGGL((bwd_dkdv_simt<64>), dim3(kv_grid), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((bwd_dkdv_simt<128>), dim3(kv_grid), dim3(512), 0, st, a);
    } else {
      if (D == 64) hipLaunchKernelGGL((bwd_dq_simt<64>), dim3(q_grid), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((bwd_dq_simt<128>), dim3(q_grid), dim3(512), 0, st, a);
    }
    return hipGetLastError();
  }
#define MATTN_PRE(DD, TAG, OF32, MODE)                                                           \
  do {                                                                                           \
    hipLaunchKernelGGL((bwd_absmax<DD, TAG, OF32>), dim3(NPART), dim3(256), 0, st, a);           \
    hipLaunchKernelGGL(bwd_scale, dim3(1), dim3(256), 0, st, a);                                 \
    hipLaunchKernelGGL((bwd_pre<DD, TAG, OF32, MODE>), dim3(pre_grid), dim3(256), 0, st, a);     \
  } while (0)
#define MATTN_BWD(DD, TAG, MODE)                                                                 \
  do {                                                                                           \
    if (stage == MATTN_BWD_PRE) {                                                                \
      if (of32) MATTN_PRE(DD, TAG, true, MODE);                                                  \
      else MATTN_PRE(DD, TAG, false, MODE);                                                      \
    } else if (stage == MATTN_BWD_DKDV) {                                                        \
      hipLaunchKernelGGL((bwd_dkdv_mfma<DD, TAG>), dim3(kv_grid), dim3(256), 0, st, a);          \
    } else {                                                                                     \
      hipLaunchKernelGGL((bwd_dq_mfma<DD, TAG>), dim3(q_grid), dim3(256), 0, st, a);             \
    }                                                                                            \
  } while (0)
  if (dtype == MATTN_BF16) {
    if (D == 64) MATTN_BWD(64, bf16_tag, 2);
    else MATTN_BWD(128, bf16_tag, 2);
  } else {
    if (D == 64) MATTN_BWD(64, f16_tag, 1);
    else MATTN_BWD(128, f16_tag, 1);
  }
#undef MATTN_BWD
#undef MATTN_PRE
  return hipGetLastError();
}

}  // namespace mattn
