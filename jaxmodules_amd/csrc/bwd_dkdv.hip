// dK/dV kernel of the masked-attention backward (the custom_vjp bwd rule,
// /root/reference/jaxmodules/attention.py:266-342): one workgroup per
// 128-key map column of (b, kv head) walking the column's present query tiles
// for every query head of the GQA group; dK and dV accumulated in registers and
// written once each -- no atomics.
#include <type_traits>

#include "common.hpp"

namespace mattn {

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
  if (item < 0 || item >= a.B * a.Hkv * a.nkt) return;  // idle slot (or an entry out of range)
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
    if (mask >= 0) mw = a.col_bits[((int64_t)mask * 2 + half) * TILE + kloc];
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
// launcher
// ---------------------------------------------------------------------------

hipError_t launch_dkdv(const KArgs& a, int D, int dtype, int grid, hipStream_t st) {
  if (dtype == MATTN_BF16) {
    if (D == 64) hipLaunchKernelGGL((bwd_dkdv_mfma<64, bf16_tag>), dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((bwd_dkdv_mfma<128, bf16_tag>), dim3(grid), dim3(256), 0, st, a);
  } else {
    if (D == 64) hipLaunchKernelGGL((bwd_dkdv_mfma<64, f16_tag>), dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((bwd_dkdv_mfma<128, f16_tag>), dim3(grid), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace mattn
