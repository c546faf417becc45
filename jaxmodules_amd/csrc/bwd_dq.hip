// dQ kernel of the masked-attention backward (the custom_vjp bwd rule,
// /root/reference/jaxmodules/attention.py:266-342): one workgroup per
// 128-query map row, dQ accumulated in registers and written once.  Every
// product runs on float16 operands.
#include <type_traits>

#include "common.hpp"

namespace mattn {

// ---------------------------------------------------------------------------
// dQ (MFMA)
// ---------------------------------------------------------------------------
// Each wave owns 32 queries.  With the float16 copies Q' = Q r, V' = V v_t
// (the forward's), dO' = dO s (bwd_pre) and K' = K k_t (the dK/dV kernel's,
// which runs first) -- r, s for the workgroup's 128-row query tile, k_t, v_t
// for each 128-key tile -- per 64-key sub-block:
//   S'^T  = K' Q'^T       (A: K' rows from LDS, B: Q'^T in registers)
//   dP'^T = V' dO'^T      (A: V' rows from LDS, B: dO'^T in registers)
//   P~    = exp2(S' c2 / (k_t r) - lse + log2(t / v_t)) = P t / v_t   (each lane owns one query)
//   dS~^T = P~^T * (dP'^T - delta s v_t) = t s dS^T
// The dP' accumulator starts at -delta s v_t instead of zero (a constant per
// lane, i.e. per query), and t / v_t is a power of two folded into P's
// exponent, so dS~ is one multiply per element.
//   dQ^T += K'^T dS~^T    (A: K'^T by transposed reads of the same K' tile)
// t is a power of two that keeps |dS~| < 2^14 (the tile bounds bwd_pre left
// in tst and the kv head's max |V|); the accumulator is in units of t s k_t,
// rescaled when the walk reaches a tile with another k_t (rare: the scales
// move in steps of 2^4).
// K' and V' are double-buffered (one array per buffer, loop unrolled by two),
// swizzled row-major tiles filled by direct global->LDS loads.  The operand
// reads are pipelined by hand (asm LDS reads one or two k-steps ahead of their
// MFMAs, counted lgkmcnt waits), and the dQ rows leave through an LDS-staged
// tile, 16 bytes per lane along each row.
// SPLIT: the kernel launched after the other dQ kernel (SPLIT = false, or
// bwd_dq_ds), which serves every row, for the split rows (srow; the
// workgroups of tiles without one return at once): it walks the tile's
// entries where a split row has an allowed key and overwrites the split rows'
// dQ.  Its products also take what float16 rounds off: dP'^T += V' dO'_lo^T
// (the rounded-off part of dO' that bwd_pre left in dol, B operands read from
// global memory four k-steps at a time) and dQ^T += K'^T dS~_lo^T, dS~_lo =
// dS~ - float16(dS~), by one more MFMA against the same K'^T operand.
// FUSED (the recomputing kernel at D = 64, where the registers allow both
// step forms in one kernel): the one dQ kernel.  A split tile walks all its
// entries with the SPLIT products and stores every row (its other rows then
// also take the rounded-off parts), the other tiles walk as SPLIT = false.
template <int D, class Tag, bool SPLIT>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))
void bwd_dq_mfma(KArgs a) {
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  using TL = TileLoad<D>;
  constexpr int BN = 64;
  constexpr int NKD = D / 16;
  constexpr int NMD = D / 32;
  constexpr int NI = D / 32;       // load instructions per wave per tile
  constexpr int BLK = 512;         // elements one load instruction fills

  // K and V tiles of one buffer in one array (V at + BN D): the V operand reads
  // reuse the K address with a constant offset
  __shared__ __attribute__((aligned(16))) uint16_t KV0[2 * BN * D], KV1[2 * BN * D];
  __shared__ __attribute__((aligned(16))) uint64_t M0[TILE], M1[TILE];

  // (the split kernel takes the launch order backwards: split tiles are
  // mostly short rows, which the order puts last)
  constexpr bool FUSED = !SPLIT && D == 64;
  const int item = a.q_order[SPLIT ? gridDim.x - 1 - blockIdx.x : blockIdx.x];
  if (item < 0 || item >= a.B * a.Hq * a.nqt) return;  // idle slot (or an entry out of range)
  if (SPLIT && !(a.asc[item] < 0.f)) return;            // no split row: the other kernel's dQ stands
  const bool fsplit = FUSED && a.asc[item] < 0.f;       // FUSED: a split tile (uniform)
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  // SPLIT: only the entries where a split row has an allowed key
  uint64_t need = ~0ull;
  int nsb = 2 * (e1 - e0);
  int ecur = e0 - 1;  // SPLIT: the entry of the last prepared sub-block

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int qloc = wave * 32 + l32;
  const int q = qt * TILE + qloc;
  const int qc = min(q, a.Lq - 1);
  const float c2 = a.scale_log2;

  u32x4 qf[NKD], df[NKD];
  // SPLIT: this lane's dO'_lo^T operands (read per use, from L1 / L2)
  const uint16_t* dlq = a.dol + (((int64_t)b * a.Hq + h) * a.nqt * TILE + q) * D + 8 * hi;
  {
    // the padded rows of the copies are zero, so q needs no clamp here
    const int64_t row = ((int64_t)b * a.Hq + h) * a.nqt * TILE + q;
    const uint16_t* qp = a.qh + row * D + 8 * hi;
    const uint16_t* dp = a.doh + row * D + 8 * hi;
#pragma unroll
    for (int kd = 0; kd < NKD; ++kd) {
      qf[kd] = *(const u32x4*)(qp + 16 * kd);
      df[kd] = *(const u32x4*)(dp + 16 * kd);
    }
  }
  if constexpr (SPLIT) {  // (after the operand loads above, whose latency it overlaps)
    need = split_entries(a, item, e0, e1, threadIdx.x & 63);
    nsb = split_subblocks(need, e0, e1);
  }
  const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + qc;
  const float nlse = -a.lse[rs];
  const float qs_r = a.qsc[item], ds_s = a.dsc[item];  // the tile's Q' and dO' scales
  const float2 ts = a.tst[item];  // (max |dO'_q|_1 of a row, max |delta s|)
  const int tb = (b * a.Hkv + hk) * a.nkt;  // first tile of this kv head in the per-tile arrays
  // t from the bound |dS s| <= max |dO'_q|_1 max |V| + max |delta s| (max |V| over the kv head)
  float vm = 0.f;
  for (int t = lane; t < a.nkt; t += 64) vm = fmaxf(vm, a.vmax[tb + t]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) vm = fmaxf(vm, __shfl_xor(vm, o));
  const float tds = pow2_scale(fmaf(ts.x, vm, ts.y), 14);
  const float ndl = -a.delta[rs];  // -delta s (delta is stored in units of s)
  const float c2r = c2 * pow2_rcp(qs_r);
  // exponent of a power of two, exactly
  auto log2p = [](float x) { return (float)((int)(__float_as_uint(x) >> 23) - 127); };
  const float nlse_t = nlse + log2p(tds);

  // float16 K' / V' rows of this kv head: dense, row stride D, padded to whole tiles
  const uint16_t* kb = a.kh + (int64_t)tb * TILE * D;
  const uint16_t* vb = a.vh + (int64_t)tb * TILE * D;
  const float* ksc = a.ksc + tb;
  const float* vsc = a.vsc + tb;
  uint32_t kld[NI];  // source byte offsets of this lane's load slots (K' and V' alike)
#pragma unroll
  for (int i = 0; i < NI; ++i) kld[i] = 2 * TL::src_off(NI * wave + i, lane, D);
  // LDS operand addresses, formed per use from lane seeds (one v_xad_u32 each)
  // rather than held in 16 registers across the loop (element offsets):
  //   row read, chunk 2 kd + hi of row l32 (+32 t):  l32 D + ((16 kd) ^ rx)
  //   K^T transposed read (mt, sec):                 tb[sec] + ((32 mt) ^ tz)
  const int rx = (8 * hi) ^ (swz<D>(l32) << 3);
  const int rrow = l32 * D;
  const int tz = 32 * (swz<D>(4 * hi + ((lane & 15) >> 2)) >> 2);
  const int tb0 = tr_src<D>(lane, 0, 0) - tz;
  const int tb1 = tr_src<D>(lane, 0, 1) - tz;
  const int wofs = __builtin_amdgcn_readfirstlane(NI * wave * BLK);
  EntryCache ec;

  // The next sub-block's loads in two parts: prep() reads its map entry before
  // the step's barrier (a wave that arrives early does it while it would wait
  // anyway), launch() issues the loads after the barrier, once the buffer
  // they fill is free.
  int nkey0 = 0, nmask = -1;  // first key and mask id of the prepared sub-block
  float nks = 1.f, nvs = 1.f;   // its tile's K' and V' scales
  auto prep = [&](int s) {
    int kt;
    int e = e0 + (s >> 1);
    if constexpr (SPLIT) {  // the next entry the split rows need
      if ((s & 1) == 0) ecur = split_next(need, ecur, e0);
      e = ecur;
    }
    ec.get(a.row_ent, e, e1, lane, kt, nmask, ksc, vsc, nks, nvs);
    nkey0 = kt * TILE + (s & 1) * BN;
  };
  auto launch = [&](int s, auto bufc) {  // global -> LDS loads of sub-block s into buffer bufc
    constexpr int BUF = decltype(bufc)::value;
    const int mask = nmask, key0 = nkey0;
    uint16_t* kl = (BUF ? KV1 : KV0) + wofs;
    uint16_t* vl = (BUF ? KV1 : KV0) + BN * D + wofs;
    if (mask >= 0) {
      const uint32_t* src = (const uint32_t*)(a.row_bits + ((int64_t)mask * 2 + (s & 1)) * TILE + wave * 32);
      __builtin_amdgcn_global_load_lds(src + lane, (__attribute__((address_space(3))) void*)((BUF ? M1 : M0) + wave * 32),
                                       4, 0, 0);
    }
    // K' and V' are padded to whole tiles: no row is out of range
    const char* kp = (const char*)(kb + (int64_t)key0 * D);
    const char* vp = (const char*)(vb + (int64_t)key0 * D);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      lds_load16(kp + kld[i], kl + i * BLK);
      lds_load16(vp + kld[i], vl + i * BLK);
    }
  };

  f32x16 acc[NMD];
#pragma unroll
  for (int i = 0; i < NMD; ++i) acc[i] = f32x16{};
  float kcur = 1.f;  // K' tile scale the accumulator is in
  // for the V' tile scale vcur: the dP' accumulators' start value -delta s
  // v_t and P~'s exponent offset -lse + log2(t / v_t); rebuilt when a tile
  // with another V' scale comes (rare)
  float vcur = 0.f, nlv = 0.f;
  f32x16 cvec = f32x16{};

  auto step = [&](auto bufc, auto spc, bool masked, float sks, float svs) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr bool SP = decltype(spc)::value;  // with the split products
    if (sks != kcur) {  // a tile with another K' scale (uniform; powers of two: exact)
      const float f = sks / kcur;
#pragma unroll
      for (int i = 0; i < NMD; ++i) acc[i] *= f;
      kcur = sks;
    }
    const float mq = c2r * pow2_rcp(sks);   // S = S' / (k_t r)
    if (svs != vcur) {  // uniform
      vcur = svs;
      nlv = nlse_t - log2p(svs);
      const float c0 = ndl * svs;
#pragma unroll
      for (int r = 0; r < 16; ++r) cvec[r] = c0;
    }
    const uint64_t mw = masked ? (BUF ? M1 : M0)[qloc] : 0;
    // operand reads pipelined by hand (asm LDS reads issued PS / PQ k-steps
    // ahead of their MFMAs, counted lgkmcnt waits); the V tile sits BN * D
    // elements after K and key half t 32 t D elements in: immediate offsets
    constexpr int PS = 1, PQ = 2;
    const uint32_t kb = lds_addr(BUF ? KV1 : KV0);
    const int rxo = opaque(rx), tzo = opaque(tz);
    const uint32_t ra = kb + 2 * (uint32_t)opaque(rrow);
    const uint32_t a0 = kb + 2 * (uint32_t)opaque(tb0), a1 = kb + 2 * (uint32_t)opaque(tb1);
    // Each 32-key half t of the sub-block is carried through S^T, dP^T, dS^T and
    // its two dQ k-steps before the next half starts (halves the live state).
    static_for<2>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      // a half whose block (the wave's 32 queries x 32 keys) is entirely
      // masked adds nothing to dQ (dS = 0): skipped
      if (masked && !__any((uint32_t)(mw >> (32 * t)) != 0u)) return;
      f32x16 st = f32x16{}, dp = cvec;
      u32x4 ka[PS + 1], va[PS + 1];
      auto rd = [&](auto kc) {
        constexpr int kd = decltype(kc)::value, sl = kd % (PS + 1);
        const uint32_t x = ra + 2 * (uint32_t)((16 * kd) ^ rxo);
        ka[sl] = ds_read128<64 * t * D>(x);
        va[sl] = ds_read128<2 * BN * D + 64 * t * D>(x);
      };
      static_for<PS>(rd);
      static_for<NKD>([&](auto kc) {
        constexpr int kd = decltype(kc)::value, sl = kd % (PS + 1);
        if constexpr (kd + PS < NKD) rd(std::integral_constant<int, kd + PS>{});
        lgkm_wait<2 * (kd + PS < NKD ? PS : NKD - 1 - kd)>();
        hold(ka[sl]);
        hold(va[sl]);
        st = H::mfma(ka[sl], qf[kd], st);
        dp = H::mfma(va[sl], df[kd], dp);
        hold(st);
        hold(dp);
      });
      if constexpr (SP) {  // dP'^T += V' dO'_lo^T, the dO'_lo^T operands loaded four at a time
        static_for<NKD / 4>([&](auto gc) {
          constexpr int g = decltype(gc)::value;
          u32x4 dl[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) dl[i] = *(const u32x4*)(dlq + 16 * (4 * g + i));
          static_for<4>([&](auto ic) {
            constexpr int i = decltype(ic)::value, kd = 4 * g + i;
            va[0] = ds_read128<2 * BN * D + 64 * t * D>(ra + 2 * (uint32_t)((16 * kd) ^ rxo));
            lgkm_wait<0>();
            hold(va[0]);
            dp = H::mfma(va[0], dl[i], dp);
            hold(dp);
          });
        });
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) st[r] = fast_exp2(fmaf(st[r], mq, nlv));
      if (masked) {
        const uint32_t w32 = (uint32_t)(mw >> (32 * t)) >> (4 * hi);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          st[r] = mask_zero(st[r], mask_ones(w32, r));
      }
      u32x4 pk[2], pl[2];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float d0 = st[r] * dp[r];
        const float d1 = st[r + 1] * dp[r + 1];
        const uint32_t w = H::pack2(d0, d1);
        pk[r >> 3][(r & 7) >> 1] = w;
        if constexpr (SP)  // the rounded-off parts (the differences are exact in float32)
          pl[r >> 3][(r & 7) >> 1] = H::pack2(d0 - H::to_f32(w & 0xffffu), d1 - H::to_f32(w >> 16));
      }
      // dQ^T += K^T dS^T over the half's two k-steps, K^T by transposed reads
      u32x2 lo[PQ + 1], up[PQ + 1];
      auto rq = [&](auto ic) {
        constexpr int i = decltype(ic)::value, mt = i / 2, ks = 2 * t + i % 2, sl = i % (PQ + 1);
        const uint32_t xm = 2 * (uint32_t)((32 * mt) ^ tzo);
        lo[sl] = ds_read_tr8<32 * ks * D>(a0 + xm);
        up[sl] = ds_read_tr8<32 * ks * D>(a1 + xm);
      };
      static_for<PQ>(rq);
      static_for<2 * NMD>([&](auto ic) {
        constexpr int i = decltype(ic)::value, mt = i / 2, kk = i % 2, sl = i % (PQ + 1);
        if constexpr (i + PQ < 2 * NMD) rq(std::integral_constant<int, i + PQ>{});
        lgkm_wait<2 * (i + PQ < 2 * NMD ? PQ : 2 * NMD - 1 - i)>();
        hold(lo[sl]);
        hold(up[sl]);
        const u32x4 aop = u32x4{lo[sl][0], lo[sl][1], up[sl][0], up[sl][1]};
        acc[mt] = H::mfma(aop, pk[kk], acc[mt]);
        hold(acc[mt]);
        if constexpr (SP) {
          acc[mt] = H::mfma(aop, pl[kk], acc[mt]);
          hold(acc[mt]);
        }
      });
    });
  };


  auto iter = [&](int s, auto bufc) {
    const bool masked = nmask >= 0;  // sub-block s, prepared one iteration ago
    const float sks = nks, svs = nvs;
    if (s + 1 < nsb) prep(s + 1);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of sub-block s have landed
    __syncthreads();                // ... and every wave's; sub-block s-1 fully consumed
    if (s + 1 < nsb) launch(s + 1, std::integral_constant<int, 1 - decltype(bufc)::value>{});
    if constexpr (FUSED) {
      if (fsplit) step(bufc, std::true_type{}, masked, sks, svs);
      else step(bufc, std::false_type{}, masked, sks, svs);
    } else {
      step(bufc, std::integral_constant<bool, SPLIT>{}, masked, sks, svs);
    }
  };
  if (nsb > 0) {
    prep(0);
    launch(0, std::integral_constant<int, 0>{});
  }
  for (int s = 0; s < nsb; s += 2) {
    iter(s, std::integral_constant<int, 0>{});
    if (s + 1 < nsb) iter(s + 1, std::integral_constant<int, 1>{});
  }

  // dQ through LDS (an eighth of the K / V buffers per wave, free once every wave is done)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint16_t* stage = (wave < 2 ? KV0 : KV1) + (wave & 1) * 32 * D;
  static_assert(2 * 32 * D <= 2 * BN * D, "output staging");
  const int r0 = qt * TILE + 32 * wave;
  store_rows<D, 2, true>(acc, a.scale * pow2_rcp(tds * ds_s * kcur), stage, a.dq,
                   (int64_t)b * a.dqs[0] + (int64_t)r0 * a.dqs[1] + (int64_t)h * a.dqs[2], a.dqs[1],
                   min(32, a.Lq - r0), lane, E::pack2, SPLIT ? a.srow[item * 4 + wave] : 0xffffffffu);
}

// ---------------------------------------------------------------------------
// dQ from the stored dS (MATTN_BWD_DS)
// ---------------------------------------------------------------------------
// The dK/dV kernel left dS~ = f s dS of every present tile as its waves held
// it (lane = key; DS_TILE layout in common.hpp), so per 64-key sub-block each
// wave only streams its four 1 KiB blocks (nontemporal direct global->LDS
// loads, 16 bytes per lane each, one sub-block ahead of use, into 4 KiB of LDS
// of its own per buffer) and turns them into B operands (lane = query) with
// ds_read_b64_tr_b16, which the blocks' chunk order makes conflict-free; it
// then runs
//   dQ^T += K'^T dS~^T    (A: K'^T by transposed reads of the K' tile in LDS)
// 2 D flop per pair instead of recomputing S and dP (another 4 D); the
// kernel streams 2 bytes per allowed pair from HBM.  Masked elements of a
// partial tile hold dS = 0, so no mask is read.  K' sub-blocks are
// double-buffered in LDS as in bwd_dq_mfma; the accumulator is in units of
// f s k_t (f s is the tile's asc), rescaled when the K' scale k_t changes.
template <int D, class Tag>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))
void bwd_dq_ds(KArgs a) {
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  using TL = TileLoad<D>;
  constexpr int BN = 64;
  constexpr int NMD = D / 32;
  constexpr int NI = D / 32;       // load instructions per wave per 64-row sub-block
  constexpr int BLK = 512;         // elements one load instruction fills

  __shared__ __attribute__((aligned(16))) uint16_t K0[BN * D], K1[BN * D];
  // per buffer and wave: one sub-block's four dS~ blocks (buffer b at byte 16384 b)
  __shared__ __attribute__((aligned(16))) uint16_t FX[2 * 4 * 2048];

  const int item = a.q_order[blockIdx.x];
  if (item < 0 || item >= a.B * a.Hq * a.nqt) return;  // idle slot (or an entry out of range)
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  const int nsb = 2 * (e1 - e0);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5;
  // the epilogue's operands, loaded here and pinned (empty asm) rather than
  // left as scalar loads in flight across the loop's hand-counted LDS waits
  const int r0 = qt * TILE + 32 * wave;
  int nrows = min(32, a.Lq - r0);  // this wave's output rows
  int64_t orow = (int64_t)b * a.dqs[0] + (int64_t)r0 * a.dqs[1] + (int64_t)h * a.dqs[2];
  int64_t ostr = a.dqs[1];
  void* odq = a.dq;
  float osc = a.scale * pow2_rcp(fabsf(a.asc[item]));  // (negative for a split tile)
  asm volatile("" : "+s"(nrows), "+s"(orow), "+s"(ostr), "+s"(odq), "+v"(osc));

  const int tb = (b * a.Hkv + hk) * a.nkt;  // first tile of this kv head in the per-tile arrays
  const uint16_t* kb = a.kh + (int64_t)tb * TILE * D;
  const float* ksc = a.ksc + tb;
  // this wave's fragments of tile e: frag + e * DS_TILE + ks * 512 (ks = 0..7)
  const uint16_t* frag = a.ds + ds_rep(a, b, h) * DS_TILE + wave * 8 * 512 + lane * 8;
  uint32_t kld[NI];  // source byte offsets of this lane's load slots
#pragma unroll
  for (int i = 0; i < NI; ++i) kld[i] = 2 * TL::src_off(NI * wave + i, lane, D);
  const int tz = 32 * (swz<D>(4 * hi + ((lane & 15) >> 2)) >> 2);
  const int tb0 = tr_src<D>(lane, 0, 0) - tz;
  const int tb1 = tr_src<D>(lane, 0, 1) - tz;
  const int wofs = __builtin_amdgcn_readfirstlane(NI * wave * BLK);
  EntryCache ec;
  // The wave's LDS blocks in each buffer (buffer u at byte 16384 u of FX):
  // block b = 2 (kk / 2) + t (32-key group kk / 2 of the sub-block, 16-query
  // half t) at 1 KiB b, chunk of lane l at 16 l.  B operand
  // of k-step kk (keys 16 kk + 4 hi + 8 j + i, i = 0..3, in slots 4 j + i) of
  // lane (query 16 t + i16, half hi): read j supplies, for lane i16 of its
  // 16-lane group, the 8 bytes of key 16 (kk % 2) + 4 hi + 8 j + i16 / 4 (of
  // the 32-key group) and queries 16 t + 4 q4 + 0..3, q4 = i16 % 4: chunk of
  // lane rl = key + 32 (q4 % 2) at position ds_pos(rl, t), bytes 8 (q4 / 2).
  // With P0 = ds_pos of the j = 0, kk = 0 lane, read (kk, j) sits at
  // byte 2048 (kk / 2) + 256 (kk % 2) + 128 (j ^ t) past P0's chunk.
  const uint32_t fxw = lds_addr(FX) + 4096 * wave;
  uint32_t fb0, fb1;  // read bases for j = 0 and j = 1
  {
    const int i16 = lane & 15, t = (lane >> 4) & 1, q4 = i16 & 3;
    const int rl = 4 * hi + (i16 >> 2) + 32 * (q4 & 1);
    const uint32_t c = fxw + 1024 * t + 16 * ds_pos(rl, 0) + 8 * (q4 >> 1);
    fb0 = c + 128 * t;
    fb1 = c + 128 * (1 - t);
  }

  // map entry of sub-block s: key tile and K' scale (s / 2 is the tile's entry)
  auto entry = [&](int s, int& kt, float& ks) {
    int m;
    float unused;
    ec.get(a.row_ent, e0 + (s >> 1), e1, lane, kt, m, ksc, ksc, ks, unused);
  };
  auto launch = [&](int s, int kt, auto bufc) {  // global -> LDS loads of sub-block s's K' rows
    constexpr int BUF = decltype(bufc)::value;
    const char* kp = (const char*)(kb + (int64_t)(kt * TILE + (s & 1) * BN) * D);
#pragma unroll
    for (int i = 0; i < NI; ++i) lds_load16(kp + kld[i], (BUF ? K1 : K0) + wofs + i * BLK);
  };
  // the four blocks of sub-block s (k-steps 4 (s % 2) .. + 3 of tile e0 + s / 2)
  // by direct global->LDS loads into buffer BUF: lane l's 16 bytes land at
  // chunk l of each block, where the reads below expect them.  Nontemporal
  // (cache policy 2): every byte is read once; temporal loads measured 4% slower.
  auto fetch = [&](int s, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const uint16_t* p = frag + (int64_t)(e0 + (s >> 1)) * DS_TILE + (s & 1) * 4 * 512;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      __builtin_amdgcn_global_load_lds(p + k * 512,
                                       (__attribute__((address_space(3))) void*)(FX + BUF * 8192 + wave * 2048 + k * 512),
                                       16, 0, 2);
  };

  f32x16 acc[NMD];
#pragma unroll
  for (int i = 0; i < NMD; ++i) acc[i] = f32x16{};
  float kcur = 1.f;  // K' tile scale the accumulator is in

  auto step = [&](auto bufc, float sks) {
    constexpr int BUF = decltype(bufc)::value;
    if (sks != kcur) {  // a tile with another K' scale (uniform; powers of two: exact)
      const float r = sks / kcur;
#pragma unroll
      for (int i = 0; i < NMD; ++i) acc[i] *= r;
      kcur = sks;
    }
    constexpr int PQ = 2, NSTEP = 4 * NMD;  // (k-step, d tile)
    const uint32_t kb0 = lds_addr(BUF ? K1 : K0);
    const int tzo = opaque(tz);
    const uint32_t a0 = kb0 + 2 * (uint32_t)opaque(tb0), a1 = kb0 + 2 * (uint32_t)opaque(tb1);
    // the sub-block's dS~ blocks read back transposed (B operands)
    u32x2 bq[4][2];
    static_for<4>([&](auto kc) {
      constexpr int kk = decltype(kc)::value, off = 16384 * BUF + 2048 * (kk / 2) + 256 * (kk % 2);
      bq[kk][0] = ds_read_tr8<off>(fb0);
      bq[kk][1] = ds_read_tr8<off>(fb1);
    });
    u32x2 lo[PQ + 1], up[PQ + 1];
    auto rq = [&](auto ic) {
      constexpr int i = decltype(ic)::value, ks = i / NMD, mt = i % NMD, sl = i % (PQ + 1);
      const uint32_t xm = 2 * (uint32_t)((32 * mt) ^ tzo);
      lo[sl] = ds_read_tr8<32 * ks * D>(a0 + xm);
      up[sl] = ds_read_tr8<32 * ks * D>(a1 + xm);
    };
    static_for<PQ>(rq);
    static_for<NSTEP>([&](auto ic) {
      constexpr int i = decltype(ic)::value, ks = i / NMD, mt = i % NMD, sl = i % (PQ + 1);
      if constexpr (i + PQ < NSTEP) rq(std::integral_constant<int, i + PQ>{});
      lgkm_wait<2 * (i + PQ < NSTEP ? PQ : NSTEP - 1 - i)>();
      if constexpr (i == 0) {  // this wait also covered the B operand reads
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          hold(bq[kk][0]);
          hold(bq[kk][1]);
        }
      }
      hold(lo[sl]);
      hold(up[sl]);
      acc[mt] = H::mfma(u32x4{lo[sl][0], lo[sl][1], up[sl][0], up[sl][1]},
                        u32x4{bq[ks][0][0], bq[ks][0][1], bq[ks][1][0], bq[ks][1][1]}, acc[mt]);
      hold(acc[mt]);
    });
  };

  // Sub-block s: its K' rows and its dS~ blocks were loaded (into buffers
  // s % 2) one iteration ahead.  Per iteration the wave waits for all its
  // loads, passes the barrier and issues the loads of s + 1 into the buffers
  // that sub-block s - 1 used.  On the 8192-query causal problem at 32 heads
  // (0.449 ms) this measured as fast as loading the blocks one sub-block
  // ahead into registers and writing them to LDS (161 against 127 registers),
  // and faster than two or three sub-blocks ahead through registers (0.485
  // and 0.470 ms).
  int nkt_ = 0;
  float nks = 1.f;  // key tile and K' scale of the prepared sub-block
  if (nsb > 0) {
    entry(0, nkt_, nks);
    launch(0, nkt_, std::integral_constant<int, 0>{});
    fetch(0, std::integral_constant<int, 0>{});
  }
  auto iter = [&](int s, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const float sks = nks;
    int kt1 = 0;
    if (s + 1 < nsb) entry(s + 1, kt1, nks);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // this wave's loads of s landed
    // every wave's K' loads of s landed; sub-block s - 1 fully consumed (each
    // wave's operand reads ended with lgkmcnt(0))
    barrier_lds();
    if (s + 1 < nsb) {
      launch(s + 1, kt1, std::integral_constant<int, 1 - BUF>{});
      fetch(s + 1, std::integral_constant<int, 1 - BUF>{});
    }
    __builtin_amdgcn_sched_barrier(0);
    step(bufc, sks);
  };
  // unrolled by two (two buffers of each): every index static
  for (int s = 0; s < nsb; s += 2) {
    iter(s, std::integral_constant<int, 0>{});
    if (s + 1 < nsb) iter(s + 1, std::integral_constant<int, 1>{});
  }

  // dQ through LDS (a quarter of the K' buffers per wave, free once every wave is done)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint16_t* stage = (wave < 2 ? K0 : K1) + (wave & 1) * 32 * D;
  static_assert(2 * 32 * D <= BN * D, "output staging");
  store_rows<D, 2, true>(acc, osc * pow2_rcp(kcur), stage, odq, orow, ostr, nrows, lane, E::pack2);
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------

template <int D, class Tag>
static void launch_dq_t(const KArgs& a, int grid, hipStream_t st) {
  // every row (from the stored dS, or recomputing), then the split rows again
  // (recomputing, with the rounded-off parts; workgroups of tiles without a
  // split row return at once).  The recomputing kernel at D = 64 serves the
  // split tiles itself.
  if (a.ds) hipLaunchKernelGGL((bwd_dq_ds<D, Tag>), dim3(grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL((bwd_dq_mfma<D, Tag, false>), dim3(grid), dim3(256), 0, st, a);
  if (a.ds || D != 64) hipLaunchKernelGGL((bwd_dq_mfma<D, Tag, true>), dim3(grid), dim3(256), 0, st, a);
}

hipError_t launch_dq(const KArgs& a, int D, int dtype, int grid, hipStream_t st) {
  if (dtype == MATTN_BF16) {
    if (D == 64) launch_dq_t<64, bf16_tag>(a, grid, st);
    else launch_dq_t<128, bf16_tag>(a, grid, st);
  } else {
    if (D == 64) launch_dq_t<64, f16_tag>(a, grid, st);
    else launch_dq_t<128, f16_tag>(a, grid, st);
  }
  return hipGetLastError();
}

}  // namespace mattn
