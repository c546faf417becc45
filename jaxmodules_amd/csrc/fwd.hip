// Forward pass of the masked attention (the custom_vjp primal,
// /root/reference/jaxmodules/attention.py:180-241, per-tile maths :52-105).
//
// cvt_v first writes V as float16 times a power of two per 128-key tile
// (vh, vsc).  Then one workgroup (4 waves) owns a 128-query map row of one
// (b, h) and walks the row's present key tiles from the block map; fully
// masked tiles are never visited.  Each wave owns 32 queries and computes, per
// 64-key sub-block,
//     S^T = K Q^T        (MFMA in the input dtype, K from LDS, Q^T in registers)
//     online softmax     (each lane owns one query, so the row max needs one
//                         cross-lane exchange and the row sum none)
//     O^T += V'^T P^T    (float16 MFMA, V'^T by transposed reads of the V' tile)
// P enters the product rounded to float16 (11 significant bits; bfloat16's 8
// leave O and the backward's delta = rowsum(dO * O) outside the 2e-3 gate on
// unit-variance inputs), and the row sum adds up exactly those rounded values,
// so that O is the exact attention output for the weights P / sum(P): then
// dP - delta = sum_j w_j (dP - dP_j) in the backward, without the rounding of
// the normaliser, which rows dominated by one key would carry into dS.
// When the backward will run, the workgroup also writes its 128 Q rows as
// float16 times a power of two (qh, qsc): they are in registers here anyway,
// and the largest attention weight of its rows (pmx: the backward splits
// float16 operands in tiles where it reaches SPLIT_P).
// K and V' are double-buffered in LDS; the next sub-block's global loads are
// in flight while the current one is computed.  K and V' tiles are moved by
// direct global->LDS loads into swizzled row-major tiles; V'^T operands are
// read with the transposing LDS read.  The operand reads are pipelined by hand
// (asm LDS reads 3 and 4 k-steps ahead of their MFMAs, counted lgkmcnt
// waits), and the output rows leave through an LDS-staged tile, 16 bytes per
// lane along each row.
#include <type_traits>

#include "common.hpp"

namespace mattn {

// V -> vh = float16 V * vsc[tile], one workgroup of 512 threads per
// (b, kv head, 128-key tile); rows past Lk are zero.  It also clears the
// tile's split-column flag, which the split rows' walk of the forward sets.
template <int D, class Tag>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void cvt_v(KArgs a) {
  __shared__ f32x2 red[8];
  // launch position -> (b, kv head, key tile), the head fastest when a row of V
  // holds all kv heads, so that the workgroups running together read whole rows
  int b, hk, kt;
  if (a.vs[2] < a.vs[1]) {
    hk = blockIdx.x % a.Hkv;
    kt = (blockIdx.x / a.Hkv) % a.nkt;
    b = blockIdx.x / (a.Hkv * a.nkt);
  } else {
    kt = blockIdx.x % a.nkt;
    hk = (blockIdx.x / a.nkt) % a.Hkv;
    b = blockIdx.x / (a.nkt * a.Hkv);
  }
  const int bh = b * a.Hkv + hk;
  const int tile = bh * a.nkt + kt;
  const int r = threadIdx.x >> 2, part = threadIdx.x & 3;
  TileRows<D> t;
  tile_load<D>(t, (const uint16_t*)a.v + (int64_t)b * a.vs[0] + (int64_t)(kt * TILE) * a.vs[1] +
                      (int64_t)hk * a.vs[2], a.vs[1], a.Lk - kt * TILE);
  const f32x2 m = block_max2_512(f32x2{tile_absmax<D, Tag>(t), 0.f}, red);
  const float s = copy_scale(m[0]);
  uint16_t* dst = a.vh + ((int64_t)bh * a.nkt * TILE + kt * TILE + r) * D;
#pragma unroll
  for (int j = 0; j < TileRows<D>::CPL; ++j)
    *(u32x4*)(dst + 8 * TileRows<D>::chunk(part, j)) = chunk_f16<Tag>(t.x[j], s);
  if (threadIdx.x == 0) {
    a.vsc[tile] = s;
    a.vmax[tile] = m[0];
    if (a.scol) a.scol[tile] = 0;
  }
}

// SPLIT: the kernel launched after the main one (SPLIT = false) for the
// split rows, the rows that put a weight of at least SPLIT_P on a key (srow;
// the workgroups of tiles without one return at once).  It walks the tile's
// entries where a split row has an allowed key again and overwrites the
// split rows' O and lse with values free of the float16 rounding of P: the
// row sum adds the unrounded weights, and O^T += V'^T P^T takes P as
// float16(P) + the rounded-off part, by one more MFMA against the same V'^T
// operand.  The backward's exp(S - lse) is then the exact softmax of these
// rows, and O the exact convex combination under it, which their split
// products need.  (The other rows of the tile keep the main kernel's O and
// lse: the entries skipped here may hold their keys.)  Where a split row has
// an allowed key in a sub-block, the walk flags that key tile's dK/dV column
// (scol), for the backward's split products.
// FUSED (the main kernel at D = 64, where the registers allow both walks in
// one kernel): a tile with split rows stores its other rows, then walks again
// as the SPLIT kernel would and stores the split rows; no second kernel is
// launched.
template <int D, class Tag, bool OUT_F32, bool SPLIT>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))
void fwd_mfma(KArgs a) {
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  using TL = TileLoad<D>;
  constexpr int BN = 64;             // keys per sub-block
  constexpr int NKD = D / 16;        // k-steps of S^T over the head dimension
  constexpr int NMD = D / 32;        // M-tiles of O^T over the head dimension
  constexpr int NI = D / 32;         // load instructions per wave per tile
  constexpr int BLK = 512;           // elements one load instruction fills
  // The running max is only raised when a row's max grows by more than 2^8
  // (base-2 units); until then P may reach 2^8, harmless in 16-bit and fp32.
  constexpr float RESCALE_SLACK = 8.f;

  // one array per buffer (K rows, then V rows): the compiler then knows the
  // loads landing in one buffer cannot alias the reads of the other
  __shared__ __attribute__((aligned(16))) uint16_t KV0[2 * BN * D], KV1[2 * BN * D];
  __shared__ __attribute__((aligned(16))) uint64_t M0[TILE], M1[TILE];  // partial-tile mask words
  __shared__ float QM[4];  // per wave: max |Q| (the float16 Q copy's scale), at the end the largest weight
  __shared__ uint32_t SR[4];  // FUSED: per wave, its split rows
  constexpr bool FUSED = !SPLIT && D == 64;
  bool swalk = false;  // FUSED: the second walk (over the split rows' entries) is running

  // (the split kernel takes the launch order backwards: split tiles are
  // mostly short rows, which the order puts last)
  const int item = a.q_order[SPLIT ? gridDim.x - 1 - blockIdx.x : blockIdx.x];
  if (item < 0 || item >= a.B * a.Hq * a.nqt) return;  // idle slot (or an entry out of range)
  if constexpr (SPLIT) {
    if (!(a.pmx[item] >= SPLIT_P)) return;  // no split row: the main kernel's O and lse stand
  }
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  const int kcol0 = (b * a.Hkv + hk) * a.nkt;  // the kv head's first dK/dV column
  // SPLIT: only the entries where a split row has an allowed key
  uint64_t need = ~0ull;
  int nsb = 2 * (e1 - e0);
  int ecur = e0 - 1;  // SPLIT: the entry of the last prepared sub-block

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the split rows' walk: this wave's split rows (bit r = row r)
  uint32_t swrow = SPLIT ? a.srow[item * 4 + wave] : 0u;
  const int l32 = lane & 31, hi = lane >> 5;
  const int qloc = wave * 32 + l32;
  const int q = qt * TILE + qloc;
  const int qc = min(q, a.Lq - 1);
  const float c2 = a.scale_log2;

  // Q^T operands: lane holds query q, head dims 16*kd + 8*hi .. +7.
  u32x4 qf[NKD];
  {
    const uint16_t* qp = (const uint16_t*)a.q + (int64_t)b * a.qs[0] + (int64_t)qc * a.qs[1] +
                         (int64_t)h * a.qs[2] + 8 * hi;
#pragma unroll
    for (int kd = 0; kd < NKD; ++kd) qf[kd] = *(const u32x4*)(qp + 16 * kd);
  }
  if constexpr (SPLIT) {  // (after the operand loads above, whose latency it overlaps)
    need = split_entries(a, item, e0, e1, threadIdx.x & 63);
    nsb = split_subblocks(need, e0, e1);
  }
  if (!SPLIT && a.qh != nullptr) {
    // float16 copy of the tile's Q rows for the backward (rows past Lq zero)
    float m = 0.f;
#pragma unroll
    for (int kd = 0; kd < NKD; ++kd)
#pragma unroll
      for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(E::to_f32(elt16(qf[kd], e))));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) QM[wave] = m;
    __syncthreads();
    const float r = copy_scale(fmaxf(fmaxf(QM[0], QM[1]), fmaxf(QM[2], QM[3])));
    uint16_t* qd = a.qh + ((int64_t)bh * a.nqt * TILE + q) * D + 8 * hi;
#pragma unroll
    for (int kd = 0; kd < NKD; ++kd)
      *(u32x4*)(qd + 16 * kd) = q < a.Lq ? chunk_f16<Tag>(qf[kd], r) : u32x4{0u, 0u, 0u, 0u};
    if (tid == 0) a.qsc[item] = r;
  }

  const uint16_t* kb = (const uint16_t*)a.k + (int64_t)b * a.ks[0] + (int64_t)hk * a.ks[2];
  // float16 V' rows of this kv head: dense, row stride D, padded to whole tiles
  const uint16_t* vb = a.vh + (int64_t)(b * a.Hkv + hk) * a.nkt * TILE * D;
  const float* vsc = a.vsc + (b * a.Hkv + hk) * a.nkt;
  uint32_t kld[NI], vld[NI];  // loop-invariant source byte offsets of this lane's load slots
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    kld[i] = 2 * TL::src_off(NI * wave + i, lane, a.ks[1]);
    vld[i] = 2 * TL::src_off(NI * wave + i, lane, D);
  }
  // LDS operand addresses, formed per use from lane seeds (element offsets):
  //   K row read, chunk 2 kd + hi of row r:  r D + ((16 kd) ^ rx),  rx = 8 hi ^ 8 swz(r)
  //   V transposed read (mt, sec):           tb[sec] + ((32 mt) ^ tz)
  const int rx = (8 * hi) ^ (swz<D>(l32) << 3);
  const int tz = 32 * (swz<D>(4 * hi + ((lane & 15) >> 2)) >> 2);
  const int tb0 = tr_src<D>(lane, 0, 0) - tz;
  const int tb1 = tr_src<D>(lane, 0, 1) - tz;

  const int wofs = __builtin_amdgcn_readfirstlane(NI * wave * BLK);  // this wave's load block
  EntryCache ec;
  // The next sub-block's loads in two parts: prep() reads its map entry before
  // the step's barrier (a wave that arrives early does it while it would wait
  // anyway), launch() issues the loads after the barrier, once the buffer
  // they fill is free.
  int nkey0 = 0, nmask = -1;  // first key and mask id of the prepared sub-block
  float nnu = 1.f;            // V' scale of the prepared sub-block's tile
  // K / V tile loads of the next sub-block on the fast path, set up by
  // launch() and issued by the step, one per S k-step, as in dK/dV.  Issued
  // together they held each wave ~800 cycles in launch() (per-wave s_memtime
  // stamps, target shape); spread out, that time moves into the MFMA phases
  // and the kernel time is unchanged to -1%.
  bool dma_on = false;
  const char* dma_kp = nullptr;
  const char* dma_vp = nullptr;
  auto dma = [&](auto bufc, auto ic) {  // load i of the sub-block that goes into buffer BUF
    constexpr int BUF = decltype(bufc)::value, i = decltype(ic)::value, k = i / 2;
    if (dma_on) {
      if constexpr (i % 2 == 0) lds_load16(dma_kp + kld[k], (BUF ? KV1 : KV0) + wofs + k * BLK);
      else lds_load16(dma_vp + vld[k], (BUF ? KV1 : KV0) + BN * D + wofs + k * BLK);
    }
  };
  auto prep = [&](int s) {
    int kt;
    float unused;
    int e = e0 + (s >> 1);
    if (SPLIT || (FUSED && swalk)) {  // the next entry the split rows need
      if ((s & 1) == 0) ecur = split_next(need, ecur, e0);
      e = ecur;
    }
    ec.get(a.row_ent, e, e1, lane, kt, nmask, vsc, vsc, nnu, unused);
    nkey0 = kt * TILE + (s & 1) * BN;
  };
  auto launch = [&](int s, auto bufc) {  // global -> LDS loads of sub-block s into buffer bufc
    constexpr int BUF = decltype(bufc)::value;
    const int mask = nmask, key0 = nkey0;
    uint16_t* kl = (BUF ? KV1 : KV0) + wofs;
    uint16_t* vl = (BUF ? KV1 : KV0) + BN * D + wofs;
    if (mask >= 0) {  // this wave's 32 mask words (256 bytes), one dword per lane
      const uint32_t* src = (const uint32_t*)(a.row_bits + ((int64_t)mask * 2 + (s & 1)) * TILE + wave * 32);
      __builtin_amdgcn_global_load_lds(src + lane, (__attribute__((address_space(3))) void*)((BUF ? M1 : M0) + wave * 32),
                                       4, 0, 0);
    }
    if (key0 + BN <= a.Lk) {  // the step issues the 2 NI tile loads
      dma_on = true;
      dma_kp = (const char*)(kb + (int64_t)key0 * a.ks[1]);
      dma_vp = (const char*)(vb + (int64_t)key0 * D);
    } else {  // ragged last sub-block: K rows past Lk re-read row Lk-1 (masked anyway); V' is padded
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int key = min(key0 + TL::row_of(NI * wave + i, lane), a.Lk - 1);
        const int c = TL::chunk_of(NI * wave + i, lane);
        lds_load16(kb + (int64_t)key * a.ks[1] + 8 * c, kl + i * BLK);
        lds_load16((const char*)(vb + (int64_t)key0 * D) + vld[i], vl + i * BLK);
      }
    }
  };

  f32x16 acc[NMD];
#pragma unroll
  for (int i = 0; i < NMD; ++i) acc[i] = f32x16{};
  float m2 = NEG_INF, l = 0.f;  // running max (base-2 units) and partial row sum
  float mtr = NEG_INF;          // the row's exact max (m2 trails it by up to RESCALE_SLACK)
  float nu = 1.f;               // V' scale the accumulators are in: acc = nu * sum P V

  auto step = [&](auto bufc, auto spc, bool masked, float snu, int skt) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr bool SP = decltype(spc)::value;  // the split rows' walk
    // operand reads pipelined by hand (asm LDS reads issued PS / PV steps ahead
    // of their MFMAs, counted lgkmcnt waits); V sits BN * D elements after K
    constexpr int PS = 3, PV = 4;
    const uint32_t kvb = lds_addr(BUF ? KV1 : KV0);
    const int rxo = opaque(rx), tzo = opaque(tz);
    const uint32_t ra = kvb + 2 * (uint32_t)opaque(l32 * D);
    // S^T = K Q^T: k-step kd reads the K rows of both 32-key halves
    f32x16 st[2] = {f32x16{}, f32x16{}};
    {
      u32x4 k0[PS + 1], k1[PS + 1];
      auto rd = [&](auto kc) {
        constexpr int kd = decltype(kc)::value, sl = kd % (PS + 1);
        const uint32_t x = ra + 2 * (uint32_t)((16 * kd) ^ rxo);
        k0[sl] = ds_read128<0>(x);
        k1[sl] = ds_read128<64 * D>(x);
      };
      static_for<PS>(rd);
      static_for<NKD>([&](auto kc) {
        constexpr int kd = decltype(kc)::value, sl = kd % (PS + 1);
        if constexpr (kd + PS < NKD) rd(std::integral_constant<int, kd + PS>{});
        lgkm_wait<2 * (kd + PS < NKD ? PS : NKD - 1 - kd)>();
        hold(k0[sl]);
        hold(k1[sl]);
        st[0] = E::mfma(k0[sl], qf[kd], st[0]);
        st[1] = E::mfma(k1[sl], qf[kd], st[1]);
        hold(st[0]);
        hold(st[1]);
        if constexpr (kd < 2 * NI) dma(std::integral_constant<int, 1 - BUF>{}, kc);
      });
      static_assert(2 * NI <= NKD, "one tile load per S k-step");
      dma_on = false;
    }
    if (masked) {
      const uint64_t mw = (BUF ? M1 : M0)[qloc];
      // a wave whose 32 rows allow no key of the sub-block (all mask words
      // zero) stops here: masked (-inf) elements would leave its softmax
      // state as it is (a pending V' rescale, a power of two, then lands at
      // the next sub-block it computes).  Its S chain ran, as it carries the
      // wave's share of the next sub-block's loads.
      if (!__any(mw != 0)) return;
      if constexpr (SP) {  // a split row of this wave with an allowed key here: flag the column
        if (__any(((swrow >> l32) & 1u) && mw != 0) && lane == 0) a.scol[kcol0 + skt] = 1;
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t w32 = (uint32_t)(mw >> (32 * t)) >> (4 * hi);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          st[t][r] = mask_neg_inf(st[t][r], mask_ones(w32, r));
      }
    }
    if constexpr (SP) {  // a full tile: every split row of the wave has allowed keys here
      if (!masked && swrow != 0u && lane == 0) a.scol[kcol0 + skt] = 1;
    }
    float mx = NEG_INF;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[t][r]);
    const float mx2 = wave_max32(mx) * c2;
    mtr = fmaxf(mtr, mx2);
    // a new V' tile scale (uniform) is folded into the same rescale
    if (snu != nu || __any(mx2 > m2 + RESCALE_SLACK)) {
      const float mn = fmaxf(m2, mx2);
      const float alpha = (mn == NEG_INF) ? 1.f : fast_exp2(m2 - mn);
      l *= alpha;
      const float aa = alpha * (snu / nu);  // powers of two: exact
#pragma unroll
      for (int i = 0; i < NMD; ++i) acc[i] *= aa;
      m2 = mn;
      nu = snu;
    }
    const float nmu = (m2 == NEG_INF) ? 0.f : -m2;
    u32x4 pk[4], plo[4];
    const f16x2 one2 = {(_Float16)1.f, (_Float16)1.f};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(fmaf(st[t][r], c2, nmu));
        const float p1 = fast_exp2(fmaf(st[t][r + 1], c2, nmu));
        const uint32_t w = H::pack2(p0, p1);
        if constexpr (SP) {  // the unrounded sum, and what float16 rounds off P
          l += p0;
          l += p1;
          plo[2 * t + (r >> 3)][(r & 7) >> 1] = H::pack2(p0 - H::to_f32(w & 0xffffu), p1 - H::to_f32(w >> 16));
        } else {
          // the row sum of the rounded values the product uses (v_dot2_f32_f16)
          l = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one2, l, false);
        }
        pk[2 * t + (r >> 3)][(r & 7) >> 1] = w;
      }
    }
    // O^T += V^T P^T, V^T operands by transposed reads of the row-major V tile;
    // step (ks, mt) feeds accumulator mt, four independent chains
    {
      const uint32_t a0 = kvb + 2 * (uint32_t)opaque(tb0), a1 = kvb + 2 * (uint32_t)opaque(tb1);
      u32x2 lo[PV + 1], up[PV + 1];
      auto rv = [&](auto ic) {
        constexpr int i = decltype(ic)::value, ks = i / NMD, mt = i % NMD, sl = i % (PV + 1);
        const uint32_t xm = 2 * (uint32_t)((32 * mt) ^ tzo);
        lo[sl] = ds_read_tr8<2 * BN * D + 32 * ks * D>(a0 + xm);
        up[sl] = ds_read_tr8<2 * BN * D + 32 * ks * D>(a1 + xm);
      };
      static_for<PV>(rv);
      static_for<4 * NMD>([&](auto ic) {
        constexpr int i = decltype(ic)::value, ks = i / NMD, mt = i % NMD, sl = i % (PV + 1);
        if constexpr (i + PV < 4 * NMD) rv(std::integral_constant<int, i + PV>{});
        lgkm_wait<2 * (i + PV < 4 * NMD ? PV : 4 * NMD - 1 - i)>();
        hold(lo[sl]);
        hold(up[sl]);
        const u32x4 aop = u32x4{lo[sl][0], lo[sl][1], up[sl][0], up[sl][1]};
        acc[mt] = H::mfma(aop, pk[ks], acc[mt]);
        hold(acc[mt]);
        if constexpr (SP) {
          acc[mt] = H::mfma(aop, plo[ks], acc[mt]);
          hold(acc[mt]);
        }
      });
    }
  };

  // sub-block s computes from buffer s % 2 while s + 1 loads into the other;
  // the loop is unrolled by two so that every buffer index is static
  auto iter = [&](int s, auto bufc, auto spc) {
    const bool masked = nmask >= 0;  // sub-block s, prepared one iteration ago
    const float snu = nnu;
    const int skt = nkey0 / TILE;    // its key tile
    if (s + 1 < nsb) prep(s + 1);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of sub-block s have landed
    __syncthreads();                // ... and every wave's; sub-block s-1 fully consumed
    if (s + 1 < nsb) launch(s + 1, std::integral_constant<int, 1 - decltype(bufc)::value>{});
    step(bufc, spc, masked, snu, skt);
  };
  auto walk = [&](auto spc) {
    if (nsb > 0) {
      prep(0);
      launch(0, std::integral_constant<int, 0>{});
      static_for<2 * NI>([&](auto ic) { dma(std::integral_constant<int, 0>{}, ic); });  // no step to carry them
      dma_on = false;
    }
    for (int s = 0; s < nsb; s += 2) {
      iter(s, std::integral_constant<int, 0>{}, spc);
      if (s + 1 < nsb) iter(s + 1, std::integral_constant<int, 1>{}, spc);
    }
  };
  const int r0 = qt * TILE + 32 * wave;
  uint16_t* stage = (wave < 2 ? KV0 : KV1) + (wave & 1) * BN * D;
  static_assert(32 * D * (OUT_F32 ? 4 : 2) <= BN * D * 2, "output staging");
  // lse and O of the rows in `keep` (the wave's 32 rows, bit r = row r), O
  // through LDS (one K / V buffer per wave, free once every wave is done)
  auto store = [&](uint32_t keep) {
    const float inv = l > 0.f ? 1.f / (l * nu) : 0.f;
    if (hi == 0 && q < a.Lq && ((keep >> l32) & 1u))
      a.lse[((int64_t)b * a.Hq + h) * a.Lq + q] = l > 0.f ? m2 + __builtin_log2f(l) : NEG_INF;
    store_rows<D, OUT_F32 ? 4 : 2, true>(acc, inv, stage, a.out,
                                   (int64_t)b * a.os[0] + (int64_t)r0 * a.os[1] + (int64_t)h * a.os[2], a.os[1],
                                   min(32, a.Lq - r0), lane, E::pack2, keep);
  };

  walk(std::integral_constant<bool, SPLIT>{});
  l = wave_sum32(l);
  // SPLIT: only the split rows' lse and O
  uint32_t keep = SPLIT ? swrow : 0xffffffffu;
  uint32_t split_rows = 0u;
  if (!SPLIT && a.pmx != nullptr) {  // the tile's largest attention weight: exp2(max - lse) of its rows
    float pm = l > 0.f ? fast_exp2(mtr - (m2 + __builtin_log2f(l))) : 0.f;
    split_rows = (uint32_t)__ballot(pm >= SPLIT_P);  // lanes 0-31: the wave's rows
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) pm = fmaxf(pm, __shfl_xor(pm, o));
    if (lane == 0) {
      QM[wave] = pm;
      if constexpr (FUSED) SR[wave] = split_rows;
      a.srow[item * 4 + wave] = split_rows;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const float tmx = fmaxf(fmaxf(QM[0], QM[1]), fmaxf(QM[2], QM[3]));
  if (!SPLIT && a.pmx != nullptr && tid == 0) a.pmx[item] = tmx;
  const bool again = FUSED && a.pmx != nullptr && tmx >= SPLIT_P;  // (uniform)
  store(again ? ~split_rows : keep);
  if constexpr (FUSED) {
    if (again) {  // the split rows' walk, as the SPLIT kernel runs it
      need = split_entries_w(a, SR[lane >> 5], SR[2 + (lane >> 5)], e0, e1, lane);
      nsb = split_subblocks(need, e0, e1);
      ecur = e0 - 1;
      swalk = true;
      swrow = split_rows;
#pragma unroll
      for (int i = 0; i < NMD; ++i) acc[i] = f32x16{};
      m2 = NEG_INF;
      l = 0.f;
      nu = 1.f;
      __syncthreads();  // every wave's staged O is read: the buffers may be refilled
      walk(std::true_type{});
      l = wave_sum32(l);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      store(split_rows);
    }
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

template <int D, class Tag>
static hipError_t launch_fwd_mfma(const KArgs& a, int grid, bool out_f32, hipStream_t st) {
  hipLaunchKernelGGL((cvt_v<D, Tag>), dim3(a.B * a.Hkv * a.nkt), dim3(512), 0, st, a);
  if (out_f32) {
    hipLaunchKernelGGL((fwd_mfma<D, Tag, true, false>), dim3(grid), dim3(256), 0, st, a);
    // split tiles again (at D = 64 the first kernel walks them again itself)
    if constexpr (D != 64) hipLaunchKernelGGL((fwd_mfma<D, Tag, true, true>), dim3(grid), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((fwd_mfma<D, Tag, false, false>), dim3(grid), dim3(256), 0, st, a);
    if constexpr (D != 64) hipLaunchKernelGGL((fwd_mfma<D, Tag, false, true>), dim3(grid), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_fwd_simt(const KArgs& a, int D, int dtype, int o_dtype, int grid, hipStream_t st);

hipError_t launch_fwd(const KArgs& a, int D, int dtype, int o_dtype, bool simt, int grid, hipStream_t st) {
  const bool of32 = (o_dtype == MATTN_F32);
  if (simt) return launch_fwd_simt(a, D, dtype, o_dtype, grid, st);
  if (dtype == MATTN_BF16)
    return D == 64 ? launch_fwd_mfma<64, bf16_tag>(a, grid, of32, st)
                   : launch_fwd_mfma<128, bf16_tag>(a, grid, of32, st);
  return D == 64 ? launch_fwd_mfma<64, f16_tag>(a, grid, of32, st)
                 : launch_fwd_mfma<128, f16_tag>(a, grid, of32, st);
}

}  // namespace mattn
