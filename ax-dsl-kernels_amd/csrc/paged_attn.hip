// Paged flash-attention decode (split-KV, GQA) and the paged KV write, for gfx950.
//
// KV cache layout (sgl_kernel_axera/attention/flash_attn.py:55): cache[P, 2, page_size, HKV, D] bf16,
// plane 0 = K, plane 1 = V. Page table in CSR form: the pages of sequence b are
// indices[indptr[b] .. indptr[b+1]); the last one holds last_page_len[b] valid tokens (1..page_size),
// every other page is full (flash_attn.py:1421-1596 page-id lookup, tail mask 87-104).
//
// Three kernels partition the work by items (a stream-K split, every workgroup taking the same number of tiles across
// (sequence, KV head) pairs, measured slower on both config 1 and the 131,072-token config 4 and was removed):
//  1. plan   — one wave: pages per split so that the number of (sequence, split, KV head) work items
//              is about one per resident split workgroup, and one descriptor per item. Depends only on the
//              page-table shape, so one plan serves every attention layer of a decode step (no host sync,
//              no memset: graph-capturable). Up to kLocalPlanBatch sequences the split and merge kernels
//              compute the same partition themselves and no plan launch is needed.
//  2. decode — persistent: a few workgroups per CU take the work items in turn. The 4 waves share every
//              16-token K/V tile of the item's pages: tiles stream HBM -> LDS by direct loads into a ring
//              and are computed in pairs (32 tokens per softmax step). Every wave computes the full scores
//              S^T = K Q^T of the pair on MFMA (Q in registers) and the online softmax in fp32 (exp2 domain),
//              then O^T += V^T P^T on MFMA for its own quarter of the head dim (V^T fragments by transposing
//              LDS reads), so no cross-wave merge is needed. A sequence with one split writes its output
//              directly; otherwise the item writes an fp32 partial (m, l, O).
//  3. merge  — per (sequence, query head) of a sequence with more than one split: log-sum-exp merge of the partials,
//              the split-KV merge of models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:330-349; zero
//              output for sequences without pages. A separate launch on purpose: merging inside the
//              decode kernel needs a device-scope release/acquire per workgroup, which on a multi-XCD
//              part writes back and invalidates the whole L2 and serialises the kernel.
#include <mutex>

#include "axk_common.h"
#include "axk_host.h"

namespace {

constexpr int kWaves = 4;
constexpr int kTile = 16;  // tokens per tile = one 16x16x16 PV MFMA k-step
constexpr int kNBufPair = 4;  // bf16 LDS ring: two tile pairs, one landing while the other is computed
constexpr int kTargetItems = 1024;
constexpr int kMaxGroup = 16;  // query heads per KV head (MFMA N tile)
constexpr float kLog2e = 1.4426950408889634f;

struct PlanHeader {
  int n_items;
  int pages_per_split;
  int bad_page;   // set to 1 if a page id outside [0, num_pages) was met (page skipped)
  int batch;      // batch / num_kv_heads the plan was made for (checked by the run kernel)
  int hkv;
  int unused;
  int pad[2];
};

// One work item: KV head kvh of sequence b, pages indices[ibeg .. ibeg + npg), split `split` of nsplit.
struct ItemDesc {
  int b, kvh, split, nsplit;
  int ibeg, npg, last_valid, pad;  // last_valid: valid tokens in the item's last page
};

size_t ws_items_max(int64_t batch, int64_t hkv) { return (size_t)kTargetItems + (size_t)batch * hkv; }

size_t ws_layout(int64_t batch, int64_t hkv, int64_t group, int64_t d, size_t* off_item, size_t* off_desc,
                 size_t* off_m, size_t* off_l, size_t* off_o) {
  const size_t maxi = ws_items_max(batch, hkv);
  size_t off = sizeof(PlanHeader);
  *off_item = off;
  off += sizeof(int) * (size_t)(batch + 1);
  off = (off + 255) & ~(size_t)255;
  *off_desc = off;
  off += sizeof(ItemDesc) * maxi;
  *off_m = off;
  off += sizeof(float) * maxi * group;
  *off_l = off;
  off += sizeof(float) * maxi * group;
  off = (off + 255) & ~(size_t)255;
  *off_o = off;
  off += sizeof(float) * maxi * group * d;
  return off;
}

constexpr int kPlanLdsBatch = 4096;  // sequences whose item offsets the plan keeps in LDS

__global__ __launch_bounds__(256) void paged_plan_kernel(const int* __restrict__ indptr,
                                                         const int* __restrict__ last_page_len, int bias, int batch,
                                                         int hkv, int page_size, int slots,
                                                         PlanHeader* __restrict__ hdr, int* __restrict__ item_off,
                                                         ItemDesc* __restrict__ descs) {
  __shared__ int s_off[kPlanLdsBatch + 1];
  __shared__ int s_ptr[kPlanLdsBatch + 1], s_last[kPlanLdsBatch];
  __shared__ int s_pps, s_items;
  const int tid = threadIdx.x, lane = tid & 63;
  const bool cached = batch <= kPlanLdsBatch;  // page table shape held in LDS: one round of global loads
  if (cached) {
    for (int b = tid; b <= batch; b += blockDim.x) {
      s_ptr[b] = indptr[b];
      if (b < batch) s_last[b] = last_page_len[b] + bias;
    }
    __syncthreads();
  }
  const int* ptr = cached ? s_ptr : indptr;
  const int* lastp = cached ? s_last : last_page_len;
  if (tid < 64) {
    int tot = 0;
    for (int b = lane; b < batch; b += 64) tot += ptr[b + 1] - ptr[b];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
    const long long work = (long long)tot * hkv;
    // one round of the persistent split kernel: at most `slots` items (each sequence may add one partial
    // split per KV head on top of work / pps), and never more than the workspace holds
    int target = min(slots, kTargetItems);
    if (target - batch * hkv >= target / 2) target -= batch * hkv;
    int pps = (int)((work + target - 1) / target);
    if (pps < 1) pps = 1;
    // prefix sum of items per sequence, 64 sequences at a time
    int base = 0;
    for (int b0 = 0; b0 < batch; b0 += 64) {
      const int b = b0 + lane;
      int cnt = 0;
      if (b < batch) cnt = hkv * ((ptr[b + 1] - ptr[b] + pps - 1) / pps);
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
      }
      if (b < batch) {
        item_off[b] = base + incl - cnt;
        if (b < kPlanLdsBatch) s_off[b] = base + incl - cnt;
      }
      base += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      item_off[batch] = base;
      if (batch <= kPlanLdsBatch) s_off[batch] = base;
      s_pps = pps;
      s_items = base;
      hdr->n_items = base;
      hdr->pages_per_split = pps;
      hdr->bad_page = 0;
      hdr->batch = batch;
      hdr->hkv = hkv;
    }
  }
  __syncthreads();
  const int pps = s_pps, n_items = s_items;
  const int* offs = batch <= kPlanLdsBatch ? s_off : item_off;  // global copy: same values, written above
  for (int it = tid; it < n_items; it += blockDim.x) {
    int lo = 0, hi = batch - 1;  // the sequence whose item range holds `it`
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (offs[mid] <= it) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int pb = ptr[b], np = ptr[b + 1] - pb;
    const int ns = (np + pps - 1) / pps;
    const int local = it - offs[b];
    const int sp = local / hkv, kvh = local - sp * hkv;  // items in (split, KV head) order
    ItemDesc d;
    d.b = b;
    d.kvh = kvh;
    d.split = sp;
    d.nsplit = ns;
    d.ibeg = pb + sp * pps;
    d.npg = min(pps, np - sp * pps);
    d.last_valid = sp == ns - 1 ? (cached ? lastp[b] : lastp[b] + bias) : page_size;
    d.pad = 0;
    descs[it] = d;
  }
}

// The bf16 cache's tile layout in LDS (also the per-wave head-dim split of every decode path).
template <int D>
struct PagedCfg {
  static constexpr int KSTEPS = D / 32;       // 16x16x32 MFMA k-steps over the head dim (QK)
  static constexpr int DW = D / kWaves;       // head-dim columns of O owned by one wave
  static constexpr int DT = DW / 16;          // 16-wide O tiles per wave
  static constexpr int RB = D * 2;            // bytes per cached row of one KV head
  static constexpr int RPI = 1024 / RB;       // rows per direct-to-LDS instruction (64 lanes x 16 B)
  static constexpr int IPP = kTile / RPI;     // instructions per plane (K or V) of a tile
  static constexpr int IPW = 2 * IPP / kWaves;  // instructions per wave per tile
  static_assert(IPW >= 1 && IPW * kWaves == 2 * IPP, "a tile's loads split evenly over the waves");
  // bytes after each 1 KiB block (bank spread for the transposing V reads)
  static constexpr int PAD = D == 256 ? 32 : 64;
  static constexpr int BLK = 1024 + PAD;
  static constexpr int PLANE = IPP * BLK;     // one plane of a tile in LDS
  static constexpr int BUF = 2 * PLANE;       // one tile (K then V)
  static AXK_DEV int row_off(int tok) { return (tok / RPI) * BLK + (tok % RPI) * RB; }
};

// The 8-bit cache decode's step (a pair of 16-token tiles per wave step) and per-lane load counts.
template <int D>
struct WaveCfg {
  static constexpr int NT = 2;                    // tiles per step
  static constexpr int RB = D;                    // bytes per cached row of one KV head
  static constexpr int NCH = RB / 16;             // 16-byte chunks per row
  static constexpr int KLT = RB / 64;             // K loads (16 B) per lane per tile
  static constexpr int KL = NT * KLT;             // ... per step (and 1 KiB V loads per tile)
  static constexpr int DTF = D / 16;              // 16-wide O^T tiles of the full head dim
  static constexpr int VPLANE = 16 * RB;          // one tile's V in a wave's slot
  static constexpr int VSLOT = NT * VPLANE;       // one step's V: each wave has two slots
  static constexpr int MERGE = kWaves * DTF * 64 * 16 + kWaves * 64 * 8;  // the end-of-item merge (over the slots)
  static constexpr int LDS = 2 * kWaves * VSLOT > MERGE ? 2 * kWaves * VSLOT : MERGE;
  static_assert(RB % 64 == 0 && 1024 % RB == 0, "a tile's V rows split evenly over 1 KiB loads");
};

// Software FP32 -> E4M3 (OCP e4m3fn) with round-to-nearest-even, as torch's float8_e4m3fn cast: |v| > 464
// (rounding to 480, past the largest finite value 448) and NaN give NaN (0x7F with the sign), values under
// 2^-6 round onto the subnormal grid m * 2^-9.
AXK_DEV uint32_t f32_to_e4m3(float v) {
  const uint32_t u = __float_as_uint(v), sgn = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
  const float av = __uint_as_float(a);
  if (a > 0x7f800000u || av > 464.0f) return sgn | 0x7fu;
  const int e = (int)(a >> 23) - 127;
  if (e < -6) return sgn | (uint32_t)rintf(av * 512.0f);  // 0 .. 8 (8 = the smallest normal, code 0x08)
  const uint32_t mant = a & 0x7fffffu;
  uint32_t m3 = mant >> 20, ex = (uint32_t)(e + 7);
  const uint32_t rb = (mant >> 19) & 1u, sticky = mant & 0x7ffffu;
  if (rb && (sticky || (m3 & 1u))) {
    if (++m3 == 8u) {
      m3 = 0u;
      ++ex;
    }
  }
  return sgn | (ex << 3) | m3;
}

typedef short axk_i16x4 __attribute__((ext_vector_type(4)));

constexpr int kLocalPlanBatch = 63;  // up to this many sequences the kernels derive the plan themselves

// The plan's partition computed by one wave from the page table (batch <= kLocalPlanBatch: lane b holds
// sequence b), with exactly the arithmetic of paged_plan_kernel: pages per split from the total work and the
// slot count, items in (sequence, split, KV head) order.
struct LocalPlan {
  int p, np, last;  // lane b: first page index, pages, last page's valid tokens of sequence b
  int off, ns;      // lane b: first item of sequence b, splits per KV head
  int pps, n_items, hkv;
};

AXK_DEV LocalPlan local_plan(const int* __restrict__ indptr, const int* __restrict__ last_page_len, int bias,
                             int batch, int hkv, int slots) {
  const int lane = threadIdx.x & 63;
  LocalPlan lp;
  lp.hkv = hkv;
  lp.p = indptr[min(lane, batch)];
  lp.last = lane < batch ? last_page_len[lane] + bias : 0;
  const int pn = __shfl(lp.p, min(lane + 1, 63), 64);
  lp.np = lane < batch ? pn - lp.p : 0;
  int tot = lp.np;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
  const long long work = (long long)tot * hkv;
  int target = min(slots, kTargetItems);
  if (target - batch * hkv >= target / 2) target -= batch * hkv;
  lp.pps = max(1, (int)((work + target - 1) / target));
  lp.ns = (lp.np + lp.pps - 1) / lp.pps;
  const int cnt = lane < batch ? hkv * lp.ns : 0;
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  lp.off = incl - cnt;
  lp.n_items = __shfl(incl, 63, 64);
  return lp;
}

// Descriptor of item `it` (< n_items) from the local plan (every lane gets the same values).
AXK_DEV ItemDesc local_item(const LocalPlan& lp, int it, int batch, int page_size) {
  const int lane = threadIdx.x & 63;
  ItemDesc d;
  // the sequence: the last lane whose first item is <= it (item ranges are consecutive; a sequence without
  // pages has an empty range and is never the last such lane for an item inside the plan)
  const unsigned long long le = __builtin_amdgcn_ballot_w64(lane < batch && lp.off <= it);
  const int b = 63 - __builtin_clzll(le);
  const int pb = __shfl(lp.p, b, 64), npb = __shfl(lp.np, b, 64), ns = __shfl(lp.ns, b, 64);
  const int local = it - __shfl(lp.off, b, 64);
  d.b = b;
  d.split = local / lp.hkv;
  d.kvh = local - d.split * lp.hkv;
  d.nsplit = ns;
  d.ibeg = pb + d.split * lp.pps;
  d.npg = min(lp.pps, npb - d.split * lp.pps);
  d.last_valid = d.split == ns - 1 ? __shfl(lp.last, b, 64) : page_size;
  d.pad = 0;
  return d;
}

// The optional attention output gate on one output value: bf16(v * sigmoid(g)) for the already bf16-rounded v (the
// elementwise sigmoid-mul of the decode layer, applied where the row is written); v as is without a gate.
AXK_DEV uint32_t gated_bf16(float v, const uint16_t* gate, int64_t gi) {
  const uint32_t vb = f32_to_bf16_bits(v);
  return gate ? f32_to_bf16_bits(bf16_bits_to_f32(vb) * sigmoid_f32(bf16_bits_to_f32(gate[gi]))) : vb;
}

// Attention of one work item over a bf16 cache. The 4 waves share every 16-token K/V tile: the tile streams HBM -> LDS
// (each wave issues a quarter of its loads) into a ring of tile pairs, computed a pair (32 tokens) at a time. Every
// wave computes the full scores S^T = K Q^T of the pair (cheap on MFMA) and the online softmax, then P x V for its
// own quarter of the head dim, so no cross-wave merge is needed. (An 8-bit cache, half the bytes per token, takes
// decode_item_8 below: there the conversions make the repeated score work too costly.)
template <int D>
__device__ __forceinline__ void decode_item(const ItemDesc& desc, int it, const uint16_t* __restrict__ q,
                                            const unsigned char* __restrict__ cache, const int* __restrict__ indices,
                                            int hq, int hkv, int page_size, int64_t num_pages, float sm_scale,
                                            PlanHeader* __restrict__ hdr,
                                            float* __restrict__ part_m, float* __restrict__ part_l,
                                            float* __restrict__ part_o, uint16_t* __restrict__ out,
                                            unsigned char* smem, const uint16_t* __restrict__ gate, int64_t ldg) {
  using C = PagedCfg<D>;  // the bf16 tile layout
  const int group = hq / hkv;
  const int b = __builtin_amdgcn_readfirstlane(desc.b), kvh = __builtin_amdgcn_readfirstlane(desc.kvh);
  const int nsplit = __builtin_amdgcn_readfirstlane(desc.nsplit);
  // the item's pages (wave-uniform: scalar registers)
  const int npg = __builtin_amdgcn_readfirstlane(desc.npg), last_valid = __builtin_amdgcn_readfirstlane(desc.last_valid);
  const int ibeg = __builtin_amdgcn_readfirstlane(desc.ibeg);
  const int tpp = page_size / kTile;  // tiles per page
  // tiles holding at least one valid token: the item's last page stops after its last valid token
  const int ntiles = npg > 0 ? (npg - 1) * tpp + min(tpp, max(0, (last_valid + kTile - 1) / kTile)) : 0;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const float c = sm_scale * kLog2e;
  const int64_t row_stride = (int64_t)hkv * D * 2;  // bytes between consecutive tokens
  const int64_t plane_stride = (int64_t)page_size * row_stride;
  const uint32_t lds0 = lds_addr(smem);

  // the item's page ids, 64 at a time: lane j holds page j of the current chunk
  int chunk = 0;
  int pid = lane < npg ? indices[ibeg + lane] : 0;

  // Q as the B operand of S^T = K Q^T: lane (head l16, group g) holds d = 32s + 8g .. +8 at step s
  axk_bf16x8 qb[C::KSTEPS];
  {
    const bool hv = l16 < group;
    const uint16_t* qp = q + ((int64_t)b * hq + kvh * group + (hv ? l16 : 0)) * D + 8 * g;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) qb[s] = hv ? load_bf16x8(qp + 32 * s) : zero_bf16x8();
  }
  // make the compiler take its waits for Q and the page ids here, before the asm loads it cannot count
  asm volatile("" : "+v"(pid));
#pragma unroll
  for (int s = 0; s < C::KSTEPS; ++s) asm volatile("" : "+v"(qb[s]));

  // tile (lp, tp) = tile tp of the item's page lp -> valid tokens and K base (both wave-uniform: scalar registers);
  // a tile past the sequence end or on a page outside the pool gets nvalid = 0 and an in-bounds base
  auto locate = [&](int lp, int tp, int& nvalid) -> const unsigned char* {
    if ((lp >> 6) != chunk) {  // wave-uniform: next 64 page ids (every 64 pages)
      chunk = lp >> 6;
      const int j = (chunk << 6) + lane;
      pid = j < npg ? indices[ibeg + j] : 0;
      asm volatile("" : "+v"(pid));  // the compiler's wait for this load stays inside this rare branch
    }
    int page = __builtin_amdgcn_readlane(pid, lp & 63);
    const int valid_in_page = (lp == npg - 1) ? last_valid : page_size;
    nvalid = min(kTile, valid_in_page - tp * kTile);
    if (page < 0 || page >= num_pages) {
      if (lane == 0 && nvalid > 0) hdr->bad_page = 1;
      page = 0;
      nvalid = 0;
    }
    return cache + (int64_t)page * 2 * plane_stride + (int64_t)(tp * kTile) * row_stride + (int64_t)kvh * D * 2;
  };
  // per-lane element offsets of this wave's loads inside a tile (token row, plane, 16-byte chunk), and the
  // same offsets clamped to row 0 for rows past nvalid
  constexpr int NCH = C::RB / 16;  // 16-byte chunks per row
  // (32-bit: the launch checks that both planes of a page span less than 2^31 bytes)
  int lane_tok[C::IPW];
  uint32_t lane_off[C::IPW], lane_off0[C::IPW];  // bytes from the tile's K base
#pragma unroll
  for (int k = 0; k < C::IPW; ++k) {
    const int j = wave * C::IPW + k;  // instruction of the tile: plane j / IPP, block j % IPP
    const int plane = j / C::IPP, blk = j - plane * C::IPP;
    lane_tok[k] = blk * C::RPI + lane / NCH;
    lane_off0[k] = (uint32_t)(plane * plane_stride + (lane % NCH) * 16);
    lane_off[k] = lane_off0[k] + (uint32_t)(lane_tok[k] * row_stride);
  }
  // the tile cursor: issue() takes the item's tiles in order (tile cur_ti = tile cur_tp of page cur_lp); past the
  // last tile it re-reads that tile and counts no tokens
  int cur_ti = 0, cur_lp = 0, cur_tp = 0;
  // this wave's share of the next tile's loads into ring buffer nb (rows past nvalid re-read row 0); returns the
  // tile's valid token count
  auto issue = [&](int nb) -> int {
    int nvalid;
    const unsigned char* kbase = locate(cur_lp, cur_tp, nvalid);
    const int nrow = nvalid > 0 ? nvalid : 1;  // every address stays inside the tile's valid rows
#pragma unroll
    for (int k = 0; k < C::IPW; ++k) {
      const int j = wave * C::IPW + k;
      const int plane = j / C::IPP, blk = j - plane * C::IPP;
      lds_dma16_so(kbase, lane_tok[k] < nrow ? lane_off[k] : lane_off0[k],
                   lds0 + nb * C::BUF + plane * C::PLANE + blk * C::BLK);
    }
    const int r = cur_ti < ntiles ? nvalid : 0;
    if (cur_ti + 1 < ntiles && ++cur_tp == tpp) {
      cur_tp = 0;
      ++cur_lp;
    }
    ++cur_ti;
    return r;
  };

  // O^T tiles: lane holds O[head l16][d = wave*DW + 16t + 4g + r] (same head layout as the softmax state)
  axk_f32x4 o[C::DT];
#pragma unroll
  for (int t = 0; t < C::DT; ++t) o[t] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // for head l16 (replicated over g and over the waves)

  // the math of a tile pair (tokens 0 .. 15 from tile a at ka, 16 .. 31 from tile b at ka + BUF; nva / nvb valid, not
  // both 0): the scores of both tiles, one online-softmax step over the 32 tokens, and O^T += V^T P^T as 32-deep
  // MFMAs. P^T's B operand (lane (head, g): tokens 8 g .. 8 g + 7) comes from the score accumulators (tokens 4 g + r
  // of each tile) by two lane swaps; V^T's A operand (lane (d, g): the same tokens) by two transposing LDS reads.
  auto pair_math = [&](const unsigned char* ka, int nva, int nvb) {
    const unsigned char* kb = ka + C::BUF;
    // a tile with no valid token (a bad page) may hold any bytes: its zero weights take the other tile's finite V
    if (nva <= 0) ka = kb;
    if (nvb <= 0) kb = ka;
    axk_f32x4 sa = axk_f32x4{0.f, 0.f, 0.f, 0.f}, sb = sa;
    const unsigned char* kra = ka + C::row_off(l16) + 16 * g;
    const unsigned char* krb = kb + C::row_off(l16) + 16 * g;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) {
      sa = mfma_bf16_16x16x32(*reinterpret_cast<const axk_bf16x8*>(kra + 64 * s), qb[s], sa);
      sb = mfma_bf16_16x16x32(*reinterpret_cast<const axk_bf16x8*>(krb + 64 * s), qb[s], sb);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      sa[rr] = (4 * g + rr < nva) ? sa[rr] * c : -INFINITY;
      sb[rr] = (4 * g + rr < nvb) ? sb[rr] * c : -INFINITY;
      mx = fmaxf(mx, fmaxf(sa[rr], sb[rr]));
    }
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx);  // finite: the pair holds at least one valid token
    const bool moved = __builtin_amdgcn_ballot_w64(m_new > m_run) != 0;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // exp2(-inf) = 0 on the first pair
    float psum = 0.f;
    axk_f32x4 pa, pb;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      pa[rr] = (4 * g + rr < nva) ? __builtin_amdgcn_exp2f(sa[rr] - m_new) : 0.f;
      pb[rr] = (4 * g + rr < nvb) ? __builtin_amdgcn_exp2f(sb[rr] - m_new) : 0.f;
      psum += pa[rr] + pb[rr];
    }
    psum = xor32_sum(xor16_sum(psum));
    l_run = l_run * alpha + psum;
    m_run = m_new;
    const axk_bf16x8 pfrag = acc_pair_to_b(pa, pb);  // P rounded to bf16 as the MFMA operand
    // V^T rows of this lane group: tokens 8 g .. 8 g + 7 = tile g / 2, rows 8 (g & 1) .. + 7
    const unsigned char* vt = (g < 2 ? ka : kb) + C::PLANE;
    const int vr = 8 * (g & 1) + (l16 >> 2);
#pragma unroll
    for (int t = 0; t < C::DT; ++t) {
      const int vc = (wave * C::DW + 16 * t + 4 * (l16 & 3)) * 2;
      const axk_i16x4 v0 = lds_read_tr16(vt + C::row_off(vr) + vc);
      const axk_i16x4 v1 = lds_read_tr16(vt + C::row_off(vr + 4) + vc);
      const axk_bf16x8 vfrag = __builtin_bit_cast(axk_bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      if (moved) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) o[t][rr] *= alpha;
      }
      o[t] = mfma_bf16_16x16x32(vfrag, pfrag, o[t]);
    }
  };

  {
    // Tile pairs: pair p = tiles 2 p, 2 p + 1 in ring slots 2 (p % 2), 2 (p % 2) + 1. Pair p + 1 is issued as pair p
    // starts, into the slots of pair p - 1 (every wave finished it before the barrier), and lands while p computes:
    // the same two tiles in flight as a single-tile ring, with one barrier, one softmax step and one set of page
    // lookups per 32 tokens. A tile past the item re-reads its last tile and counts no tokens.
    const int npairs = (ntiles + 1) / 2;
    int nva = issue(0), nvb = issue(1);
    for (int pp = 0; pp < npairs; ++pp) {
      const int sl = 2 * (pp & 1);
      wait_vmcnt<0>();                 // this wave's loads of pair pp have landed
      __builtin_amdgcn_s_barrier();    // ... and every other wave's; all are done with pair pp - 1
      int nna = 0, nnb = 0;
      if (pp + 1 < npairs) {           // uniform
        nna = issue(2 - sl);  // tiles 2 pp + 2, 2 pp + 3
        nnb = issue(3 - sl);
      }
      if (nva > 0 || nvb > 0) pair_math(smem + sl * C::BUF, nva, nvb);  // uniform over the workgroup
      nva = nna;
      nvb = nnb;
    }
  }
  wait_vmcnt<0>();  // every load has landed before the buffers are reused
  __builtin_amdgcn_s_barrier();

  // every wave holds the same (m, l) for head l16 and O^T for its own columns
  const int64_t out_base = ((int64_t)b * hq + kvh * group) * D;
  const bool hv = l16 < group;
  if (nsplit == 1) {  // the whole sequence in one item: normalise and store
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    const int64_t gi0 = ((int64_t)b * hq + kvh * group + l16) * ldg;  // this lane's head's gate row
#pragma unroll
    for (int t = 0; t < C::DT; ++t) {
      if (!hv) continue;
      const int col = wave * C::DW + 16 * t + 4 * g;
      uint2 w;
      w.x = gated_bf16(o[t][0] * inv, gate, gi0 + col) | (gated_bf16(o[t][1] * inv, gate, gi0 + col + 1) << 16);
      w.y = gated_bf16(o[t][2] * inv, gate, gi0 + col + 2) | (gated_bf16(o[t][3] * inv, gate, gi0 + col + 3) << 16);
      *reinterpret_cast<uint2*>(out + out_base + (int64_t)l16 * D + col) = w;
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
    if (hv)
      *reinterpret_cast<float4*>(part_o + ((int64_t)it * group + l16) * D + wave * C::DW + 16 * t + 4 * g) =
          make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
  if (wave == 0 && lane < group) {
    part_m[(int64_t)it * group + lane] = m_run;
    part_l[(int64_t)it * group + lane] = l_run;
  }
}

// Attention of one work item over an 8-bit cache (FP8 E4M3 codes * inv_scale, exact for a power-of-two scale, on bf16
// MFMAs; QM = 1: INT8 codes q times s, the bf16 scale of the row and KV head in kv_scales [pages, 2, page, hkv],
// q35_group.py kv_page 208-221, on fp16 MFMAs: the codes enter exactly as 1152 + q by one byte permute per two codes,
// the row scales multiply the scores (K) and the probabilities (V) instead of every element, and the constant
// offsets come off the sums; the reference rounds bf16(q * s) per element, this rounds only the products' fp32
// sums and the fp16 probabilities), the item's tiles split between the 4 waves. A step is a pair of 16-token tiles
// (16 KiB of K and V at D = 256); wave w streams steps [ns w / 4, ns (w + 1) / 4) of the item's ns steps with its own
// online softmax, so every stored byte is converted once (no score or softmax work is repeated across waves): K
// straight into registers (lane (token l16, g) loads the 16-byte row chunks 64 s' + 16 g of its MFMA A operand), V by
// direct loads into the wave's LDS slot (chunk c of row r at chunk slot c ^ (r mod NCH), so the transposing 8-bit reads
// spread over the banks), read back transposed as the A operand of O^T += V^T P^T. The next step's loads are issued
// before the current step is computed; no barrier while streaming. At the end the four (m, l, O) are merged through
// LDS and each wave finishes a quarter of the head dim.
template <int D, int QM>
__device__ __forceinline__ void decode_item_8(const ItemDesc& desc, int it, const uint16_t* __restrict__ q,
                                              const unsigned char* __restrict__ cache,
                                              const int* __restrict__ indices, int hq, int hkv, int page_size,
                                              int64_t num_pages, float sm_scale, float inv_scale,
                                              const unsigned char* __restrict__ kv_scales,
                                              PlanHeader* __restrict__ hdr, float* __restrict__ part_m,
                                              float* __restrict__ part_l, float* __restrict__ part_o,
                                              uint16_t* __restrict__ out, unsigned char* smem) {
  using C = PagedCfg<D>;  // each wave's final quarter of the head dim
  using W = WaveCfg<D>;
  constexpr int NT = W::NT, RB = W::RB, NCH = W::NCH, KLT = W::KLT, KL = W::KL, DTF = W::DTF;
  const int group = hq / hkv;
  const int b = __builtin_amdgcn_readfirstlane(desc.b), kvh = __builtin_amdgcn_readfirstlane(desc.kvh);
  const int nsplit = __builtin_amdgcn_readfirstlane(desc.nsplit);
  const int npg = __builtin_amdgcn_readfirstlane(desc.npg), last_valid = __builtin_amdgcn_readfirstlane(desc.last_valid);
  const int ibeg = __builtin_amdgcn_readfirstlane(desc.ibeg);
  const int tpp = page_size / kTile;  // tiles per page
  // tiles holding at least one valid token: the item's last page stops after its last valid token
  const int ntiles = npg > 0 ? (npg - 1) * tpp + min(tpp, max(0, (last_valid + kTile - 1) / kTile)) : 0;
  const int nsteps = (ntiles + NT - 1) / NT;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const float c = sm_scale * kLog2e;
  const int64_t row_stride = (int64_t)hkv * RB;  // bytes between consecutive tokens
  const int64_t plane_stride = (int64_t)page_size * row_stride;
  const int s_beg = (nsteps * wave) >> 2, s_end = (nsteps * (wave + 1)) >> 2;

  // Q as the B operand of S^T = K Q^T: K is read as 16-byte row chunks (16 d), so lane (head l16, group g) holds
  // d = 64s' + 16g + 8e .. +8 at k-step 2s' + e, e = 0, 1
  axk_bf16x8 qb[C::KSTEPS];
  {
    const bool hv = l16 < group;
    const uint16_t* qp = q + ((int64_t)b * hq + kvh * group + (hv ? l16 : 0)) * D + 16 * g;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) qb[s] = hv ? load_bf16x8(qp + 64 * (s >> 1) + 8 * (s & 1)) : zero_bf16x8();
  }
  // INT8 (QM = 1) runs its MFMAs on fp16: Q scaled per head by a power of two qs that puts its largest magnitude in
  // [2^14, 2^15) (bf16 -> fp16 then keeps every bit of each element down to 2^-10 of that magnitude), the codes as
  // exact fp16 1152 + code (i8x8_to_f16x8_off), so a score accumulates S' = sum q (1152 + code) and its code part is
  // S' - qoff with qoff = 1152 * (the head's fp16 Q summed); the K row scale and cq = the softmax scale / qs follow
  float qoff = 0.f, cq = c;
  axk_f16x8 qh[QM == 1 ? C::KSTEPS : 1];
  if constexpr (QM == 1) {
    float amax = 0.f;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)qb[s][e]));
    amax = xor32_max(xor16_max(amax));  // the head's (lanes l16, l16 + 16, + 32, + 48)
    const int ex = amax > 0.f ? max(-120, min(120, ilogbf(amax))) : 0;
    const float qs = ldexpf(1.0f, 14 - ex);
    float qsum = 0.f;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 h = (_Float16)((float)qb[s][e] * qs);
        qh[s][e] = h;
        qsum += (float)h;
      }
    qoff = 1152.0f * xor32_sum(xor16_sum(qsum));
    cq = c * ldexpf(1.0f, ex - 14);
  }

  // the tile cursor: tiles are taken in order (tile cur_ti = tile cur_tp of the item's page cur_lp); past the item's
  // last tile it re-reads that tile and counts no tokens
  int cur_ti = s_beg * NT;
  int cur_lp = cur_ti / tpp, cur_tp = cur_ti - cur_lp * tpp;
  // the item's page ids, 64 at a time: lane j holds page j of the current chunk
  int chunk = cur_lp >> 6;
  int pid = (chunk << 6) + lane < npg ? indices[ibeg + (chunk << 6) + lane] : 0;
  // tile (lp, tp) -> valid tokens and its K base (both wave-uniform); a tile on a page outside the pool gets
  // nvalid = 0 and an in-bounds base (page 0); QM: sbase = the tile's row scales, plane 0
  auto locate = [&](int lp, int tp, int& nvalid, const unsigned char*& sbase) -> const unsigned char* {
    if ((lp >> 6) != chunk) {  // wave-uniform: next 64 page ids (every 64 pages)
      chunk = lp >> 6;
      const int j = (chunk << 6) + lane;
      pid = j < npg ? indices[ibeg + j] : 0;
    }
    int page = __builtin_amdgcn_readlane(pid, lp & 63);
    const int valid_in_page = (lp == npg - 1) ? last_valid : page_size;
    nvalid = min(kTile, valid_in_page - tp * kTile);
    if (page < 0 || page >= num_pages) {
      if (lane == 0 && nvalid > 0) hdr->bad_page = 1;
      page = 0;
      nvalid = 0;
    }
    if constexpr (QM == 1) sbase = kv_scales + ((int64_t)page * 2 * page_size + tp * kTile) * hkv * 2;
    return cache + (int64_t)page * 2 * plane_stride + (int64_t)(tp * kTile) * row_stride + (int64_t)kvh * RB;
  };

  // one step: K (tile j, chunk s': k[j KLT + s']) and (QM) the scales of this lane's K row (ks[j]) and of the eight V
  // rows its transposing reads return (vs) into registers by ordinary loads; V by direct loads into the wave's LDS
  // slot (asm: the compiler counts none of them; wait_step waits for everything)
  struct Step {
    axk_u32x4 k[KL];
    int nv[NT];
    float ks[NT];
    float vs[8];
  };
  // per-lane V load offsets inside a tile (token row, 16-byte chunk: lane slot q of row r loads chunk q ^ (r mod NCH)),
  // and the same clamped to row 0 for rows past nvalid
  constexpr int VPT = KLT;  // V loads per tile (1 KiB each)
  int vtok[VPT];
  uint32_t voff[VPT], voff0[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    vtok[i] = i * (64 / NCH) + lane / NCH;
    const int ch = (lane % NCH) ^ (vtok[i] % NCH);
    voff0[i] = (uint32_t)(plane_stride + 16 * ch);
    voff[i] = voff0[i] + (uint32_t)(vtok[i] * row_stride);
  }
  const uint32_t lds_slots = lds_addr(smem) + wave * 2 * W::VSLOT;
  // this lane's K row offset (token l16, chunk g) and the same for row 0; QM: the V scales' plane (plane 1, head kvh)
  const uint32_t k_off = (uint32_t)(l16 * row_stride + 16 * g), k_off0 = (uint32_t)(16 * g);
  const uint32_t ks_off = (uint32_t)((l16 * hkv + kvh) * 2), ks_off0 = (uint32_t)(kvh * 2);
  const uint32_t vs_off0 = (uint32_t)(page_size * hkv * 2 + kvh * 2);
  // QM: the scales of KV head kvh in rows 4 g .. 4 g + 3 from p = their row 4 g, head 0: one 8- or 16-byte load for
  // one or two KV heads (rows at hkv * 2 bytes) when the scale array is that aligned, four 2-byte loads otherwise;
  // packed (rows 4 g, + 1), (+ 2, + 3)
  const uint32_t row4_off = (uint32_t)(4 * g * hkv * 2);
  const bool svec = (reinterpret_cast<uintptr_t>(kv_scales) & (hkv == 1 ? 7u : 15u)) == 0;
  auto load_scales4 = [&](const unsigned char* p, uint32_t& lo, uint32_t& hi) {
    if (svec && hkv == 1) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      lo = v.x;
      hi = v.y;
    } else if (svec && hkv == 2) {  // dword i = (row i, head 0) | (row i, head 1) << 16
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      const uint32_t sel = kvh ? 0x07060302u : 0x05040100u;
      lo = __builtin_amdgcn_perm(v.y, v.x, sel);
      hi = __builtin_amdgcn_perm(v.w, v.z, sel);
    } else {
      const uint16_t* q2 = reinterpret_cast<const uint16_t*>(p) + kvh;
      lo = (uint32_t)q2[0] | ((uint32_t)q2[hkv] << 16);
      hi = (uint32_t)q2[2 * hkv] | ((uint32_t)q2[3 * hkv] << 16);
    }
  };
  auto issue_step = [&](Step& st, int sl) {
    const unsigned char* sbs[NT];
    int nrows[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      int nvalid;
      const unsigned char* sb = nullptr;
      const unsigned char* base = locate(cur_lp, cur_tp, nvalid, sb);
      st.nv[j] = cur_ti < ntiles ? nvalid : 0;
      const int nrow = nvalid > 0 ? nvalid : 1;  // every address stays inside the tile's valid rows
      sbs[j] = sb;
      nrows[j] = nrow;
      if (cur_ti + 1 < ntiles && ++cur_tp == tpp) {
        cur_tp = 0;
        ++cur_lp;
      }
      ++cur_ti;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        lds_dma16_so(base, vtok[i] < nrow ? voff[i] : voff0[i],
                     lds_slots + sl * W::VSLOT + j * W::VPLANE + i * 1024);
      const bool krow = l16 < nrow;
      const unsigned char* kp = base + (krow ? k_off : k_off0);
#pragma unroll
      for (int s = 0; s < KLT; ++s)
        st.k[j * KLT + s] = __builtin_nontemporal_load(reinterpret_cast<const axk_u32x4*>(kp + 64 * s));
      if constexpr (QM == 1)
        st.ks[j] = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(sb + (krow ? ks_off : ks_off0)));
    }
    if constexpr (QM == 1) {
      const uint32_t hs = (uint32_t)(hkv * 2);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int tl = jj >> 2, row = 4 * g + (jj & 3);
        const unsigned char* sbt = tl ? sbs[1] : sbs[0];
        const bool in = row < (tl ? nrows[1] : nrows[0]);
        const float x = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(sbt + vs_off0 + (in ? row * hs : 0u)));
        st.vs[jj] = (tl ? st.nv[1] : st.nv[0]) > 0 ? x : 0.f;
      }
    }
  };
  // every load of the step has landed (the register values pass through the wait, so the compiler adds none later)
  auto wait_step = [&](Step& st) {
    wait_vmcnt<0>();
#pragma unroll
    for (int i = 0; i < KL; ++i) asm volatile("" : "+v"(st.k[i]));
    if constexpr (QM == 1) {
#pragma unroll
      for (int j = 0; j < NT; ++j) asm volatile("" : "+v"(st.ks[j]));
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) asm volatile("" : "+v"(st.vs[jj]));
    }
  };

  // FP8: 8 stored bytes -> 8 bf16 (4 dwords), code * inv_scale
  auto cvt8 = [&](uint32_t w0, uint32_t w1) -> axk_bf16x8 {
    const axk_u32x4 r = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, inv_scale, false)),
                         __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, inv_scale, true)),
                         __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, inv_scale, false)),
                         __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, inv_scale, true))};
    return __builtin_bit_cast(axk_bf16x8, r);
  };

  // O^T over the full head dim: lane holds O[head l16][d = 16t + 4g + r]
  axk_f32x4 o[DTF];
#pragma unroll
  for (int t = 0; t < DTF; ++t) o[t] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // for head l16 (replicated over g)
  // INT8: P'^T = P^T times the V-row scales times 2^-e_run (e_run: the largest scale exponent seen by the wave, so
  // P' <= 2 in fp16), against the codes as 1152 + code; o_one accumulates sum P' (an all-ones A operand: exactly the
  // P' the MFMAs saw), so O = (O' - 1152 sum P') 2^e_run at the end
  axk_f32x4 o_one = {0.f, 0.f, 0.f, 0.f};
  int e_run = -1000;

  // the math of one step whose V is in the slot (at least one valid token)
  auto compute = [&](const Step& st, int sl) {
    const unsigned char* slot = smem + (wave * 2 + sl) * W::VSLOT;
    axk_f32x4 sc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      sc[j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KLT; ++s) {
        const axk_u32x4 w = st.k[j * KLT + s];
        if constexpr (QM == 1) {
          sc[j] = mfma_f16_16x16x32(i8x8_to_f16x8_off(w[0], w[1]), qh[2 * s], sc[j]);
          sc[j] = mfma_f16_16x16x32(i8x8_to_f16x8_off(w[2], w[3]), qh[2 * s + 1], sc[j]);
        } else {
          sc[j] = mfma_bf16_16x16x32(cvt8(w[0], w[1]), qb[2 * s], sc[j]);
          sc[j] = mfma_bf16_16x16x32(cvt8(w[2], w[3]), qb[2 * s + 1], sc[j]);
        }
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float v;
        if constexpr (QM == 1) {
          v = (sc[j][rr] - qoff) * (__shfl(st.ks[j], 4 * g + rr, 64) * cq);
        } else
          v = sc[j][rr] * c;
        sc[j][rr] = (4 * g + rr < st.nv[j]) ? v : -INFINITY;
        mx = fmaxf(mx, sc[j][rr]);
      }
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(m_run, mx);  // finite: the step holds at least one valid token
    int e_new = e_run;
    float vs[8];  // QM: the V row scales of this lane's score rows (jj < 4: tile 0 row 4 g + jj, else tile 1), 0 past
                  // a tile's valid rows (whatever bytes lie there)
    if constexpr (QM == 1) {  // the step's largest V-row scale exponent (a valid tile's scales are > 0)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) vs[jj] = st.vs[jj];
      float vm = 0.f;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) vm = fmaxf(vm, vs[jj]);
      vm = wave_max(vm);
      if (vm > 0.f) e_new = max(e_run, ilogbf(vm));
      e_new = __builtin_amdgcn_readfirstlane(e_new);
    }
    // the running max rarely moves after the first steps: rescale O only when it did (wave-uniform test)
    const bool moved = __builtin_amdgcn_ballot_w64(m_new > m_run) != 0 || e_new != e_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // exp2(-inf) = 0 on the first step
    float psum = 0.f;
    axk_f32x4 p[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        p[j][rr] = (4 * g + rr < st.nv[j]) ? __builtin_amdgcn_exp2f(sc[j][rr] - m_new) : 0.f;
        psum += p[j][rr];
      }
    psum = xor32_sum(xor16_sum(psum));
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (moved) {
      const float f = QM == 1 ? alpha * ldexpf(1.0f, e_run - e_new) : alpha;  // 2^(e_run - e_new): 0 at the start
#pragma unroll
      for (int t = 0; t < DTF; ++t)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) o[t][rr] *= f;
      if constexpr (QM == 1) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) o_one[rr] *= f;
      }
    }
    e_run = e_new;
    // the 32-deep step: P^T's B operand from both score tiles by two lane swaps; V^T's A operand (lane (d, g):
    // tokens 8 g .. 8 g + 7 = tile g / 2, rows 8 (g & 1) .. + 7) by one transposing 8-bit read per 16 columns
    // (source lane 2j + a: row 8 (g & 1) + j, bytes 8a .. 8a + 7 of the chunk; lane i receives column i). A tile
    // without a valid token (a bad page: any bytes) is read from the other tile, with zero weights.
    int tv = g >= 2 ? 1 : 0;
    if (st.nv[tv] <= 0) tv = 1 - tv;
    const int vr = 8 * (g & 1) + (l16 >> 1);
    const unsigned char* vrow = slot + tv * W::VPLANE + vr * RB + 8 * (l16 & 1);
    const int vsw = vr % NCH;
    if constexpr (QM == 1) {
      const float ef = ldexpf(1.0f, -e_run);
      axk_f32x4 pa, pb;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        pa[rr] = p[0][rr] * (vs[rr] * ef);
        pb[rr] = p[1][rr] * (vs[4 + rr] * ef);
      }
      const axk_f16x8 pfh = acc_pair_to_b_f16(pa, pb);
#pragma unroll
      for (int t = 0; t < DTF; ++t) {
        const axk_i32x2 w = lds_read_tr8(vrow + 16 * (t ^ vsw));
        o[t] = mfma_f16_16x16x32(i8x8_to_f16x8_off((uint32_t)w[0], (uint32_t)w[1]), pfh, o[t]);
      }
      const axk_u32x4 ones = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};  // fp16 1.0 x 8
      o_one = mfma_f16_16x16x32(__builtin_bit_cast(axk_f16x8, ones), pfh, o_one);
    } else {
      const axk_bf16x8 pfrag = acc_pair_to_b(p[0], p[1]);
#pragma unroll
      for (int t = 0; t < DTF; ++t) {
        const axk_i32x2 w = lds_read_tr8(vrow + 16 * (t ^ vsw));
        o[t] = mfma_bf16_16x16x32(cvt8((uint32_t)w[0], (uint32_t)w[1]), pfrag, o[t]);
      }
    }
  };

  auto any_valid = [&](const Step& st) {
    bool a = false;
#pragma unroll
    for (int j = 0; j < NT; ++j) a = a || st.nv[j] > 0;
    return a;
  };
  Step sa, sb;
  if (s_beg < s_end) issue_step(sa, 0);
  for (int s = s_beg; s < s_end; s += 2) {  // uniform
    wait_step(sa);
    if (s + 1 < s_end) issue_step(sb, 1);  // the next step's loads fly while this one is computed
    if (any_valid(sa)) compute(sa, 0);
    if (s + 1 >= s_end) break;
    wait_step(sb);
    if (s + 2 < s_end) issue_step(sa, 0);
    if (any_valid(sb)) compute(sb, 1);
  }

  if constexpr (QM == 1) {  // O = (O' - 1152 sum P') 2^e_run (a wave without tokens: all zero)
    const float r = 1152.0f * o_one[0], ef = e_run > -1000 ? ldexpf(1.0f, e_run) : 0.f;
#pragma unroll
    for (int t = 0; t < DTF; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) o[t][rr] = (o[t][rr] - r) * ef;
  }

  // merge the four waves' (m, l, O^T) through LDS (over the V slots): wave w takes the head-dim quarter
  // [w D / 4, (w + 1) D / 4)
  __syncthreads();  // every wave is done with its slot
  float* mo = reinterpret_cast<float*>(smem);      // [wave][t][lane][4]
  float* ml = mo + kWaves * DTF * 64 * 4;          // [wave][lane][2]
#pragma unroll
  for (int t = 0; t < DTF; ++t) *reinterpret_cast<axk_f32x4*>(mo + ((wave * DTF + t) * 64 + lane) * 4) = o[t];
  ml[(wave * 64 + lane) * 2] = m_run;
  ml[(wave * 64 + lane) * 2 + 1] = l_run;
  __syncthreads();
  float mw[kWaves], lw[kWaves];
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    mw[w] = ml[(w * 64 + lane) * 2];
    lw[w] = ml[(w * 64 + lane) * 2 + 1];
    M = fmaxf(M, mw[w]);
  }
  float fw[kWaves];
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    fw[w] = mw[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);  // a wave without tokens: -inf, 0
    L += fw[w] * lw[w];
  }
  axk_f32x4 of[C::DT];
#pragma unroll
  for (int t = 0; t < C::DT; ++t) {
    of[t] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const axk_f32x4 x = *reinterpret_cast<const axk_f32x4*>(mo + ((w * DTF + wave * C::DT + t) * 64 + lane) * 4);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) of[t][rr] += fw[w] * x[rr];
    }
  }

  // (M, L) for head l16 and O^T for this wave's columns d = wave DW + 16t + 4g + r
  const int64_t out_base = ((int64_t)b * hq + kvh * group) * D;
  const bool hv = l16 < group;
  if (nsplit == 1) {  // the whole sequence in one item: normalise and store
    const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
    for (int t = 0; t < C::DT; ++t) {
      if (!hv) continue;
      uint2 w;
      w.x = f32_to_bf16_bits(of[t][0] * inv) | (f32_to_bf16_bits(of[t][1] * inv) << 16);
      w.y = f32_to_bf16_bits(of[t][2] * inv) | (f32_to_bf16_bits(of[t][3] * inv) << 16);
      *reinterpret_cast<uint2*>(out + out_base + (int64_t)l16 * D + wave * C::DW + 16 * t + 4 * g) = w;
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
    if (hv)
      *reinterpret_cast<float4*>(part_o + ((int64_t)it * group + l16) * D + wave * C::DW + 16 * t + 4 * g) =
          make_float4(of[t][0], of[t][1], of[t][2], of[t][3]);
  if (wave == 0 && lane < group) {
    part_m[(int64_t)it * group + lane] = M;
    part_l[(int64_t)it * group + lane] = L;
  }
}

// Persistent split kernel: a few workgroups per CU; workgroup w takes items w, w + gridDim.x, ... (the plan
// sizes the items to about one per workgroup). With local != 0 the descriptors come from the page table
// directly (local_plan), otherwise from the plan in the workspace.
template <int D, int KB, int QM = 0>
__global__ __launch_bounds__(256, KB == 1 ? 2 : 1) void paged_decode_kernel(
    const uint16_t* __restrict__ q, const unsigned char* __restrict__ cache, const int* __restrict__ indptr,
    const int* __restrict__ last_page_len, const int* __restrict__ indices, int batch, int hq, int hkv,
    int page_size, int64_t num_pages, float sm_scale, float inv_scale, const unsigned char* __restrict__ kv_scales,
    int local, int bias,
    PlanHeader* __restrict__ hdr, const ItemDesc* __restrict__ descs, float* __restrict__ part_m,
    float* __restrict__ part_l, float* __restrict__ part_o, uint16_t* __restrict__ out,
    const uint16_t* __restrict__ gate, int64_t ldg) {
  extern __shared__ __align__(16) unsigned char smem[];
  if (local) {
    const LocalPlan lp = local_plan(indptr, last_page_len, bias, batch, hkv, gridDim.x);
    for (int it = blockIdx.x; it < lp.n_items; it += gridDim.x) {
      const ItemDesc desc = local_item(lp, it, batch, page_size);
      if constexpr (KB == 2)
        decode_item<D>(desc, it, q, cache, indices, hq, hkv, page_size, num_pages, sm_scale, hdr, part_m, part_l,
                       part_o, out, smem, gate, ldg);
      else
        decode_item_8<D, QM>(desc, it, q, cache, indices, hq, hkv, page_size, num_pages, sm_scale, inv_scale,
                             kv_scales, hdr, part_m, part_l, part_o, out, smem);
      __syncthreads();  // LDS is reused by the next item
    }
    return;
  }
  // the header and the first descriptor are independent loads: one round trip (the descriptor slot exists
  // whatever the plan holds, gridDim.x <= the workspace's item capacity)
  const PlanHeader h = *hdr;
  ItemDesc desc = descs[blockIdx.x];
  if (h.batch != batch || h.hkv != hkv) return;
  for (int it = blockIdx.x; it < h.n_items; it += gridDim.x) {
    if (it != (int)blockIdx.x) desc = descs[it];
    if constexpr (KB == 2)
      decode_item<D>(desc, it, q, cache, indices, hq, hkv, page_size, num_pages, sm_scale, hdr, part_m, part_l,
                     part_o, out, smem, gate, ldg);
    else
      decode_item_8<D, QM>(desc, it, q, cache, indices, hq, hkv, page_size, num_pages, sm_scale, inv_scale,
                           kv_scales, hdr, part_m, part_l, part_o, out, smem);
    __syncthreads();
  }
}

// One wave per (sequence, query head), four per workgroup: log-sum-exp merge of the item partials of a sequence with
// more than one split; zero output for a sequence without pages. Splits are taken 16 at a time: lane j loads split
// j's (m, l) while every lane loads its D / 64 columns of the 16 splits' O (all of a pass issued before any is used,
// the O loads independent of m), then one running (m, l, O) per wave; no LDS, no barrier.
template <int D>
__global__ __launch_bounds__(256) void paged_merge_kernel(const int* __restrict__ indptr,
                                                          const int* __restrict__ last_page_len,
                                                          PlanHeader* __restrict__ hdr,
                                                          const int* __restrict__ item_off, int batch, int hq,
                                                          int hkv, int slots, int local, int bias,
                                                          const float* __restrict__ part_m,
                                                          const float* __restrict__ part_l,
                                                          const float* __restrict__ part_o,
                                                          uint16_t* __restrict__ out,
                                                          const uint16_t* __restrict__ gate, int64_t ldg) {
  constexpr int V = D / 64;  // output columns per lane
  constexpr int P = 16;      // splits per pass
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int bh = blockIdx.x * 4 + wave;
  if (bh >= batch * hq) return;  // a whole wave
  const int b = bh / hq, h = bh - b * hq;
  const int group = hq / hkv, kvh = h / group, hh = h - kvh * group;
  int np, nsplit, i0;
  if (local) {
    const LocalPlan lp = local_plan(indptr, last_page_len, bias, batch, hkv, slots);
    np = __shfl(lp.np, b, 64);
    nsplit = __shfl(lp.ns, b, 64);
    i0 = __shfl(lp.off, b, 64) + kvh;
  } else {
    // header, page range and item range: independent loads, one round trip
    const int hb = hdr->batch, hk = hdr->hkv;
    const int p0 = indptr[b], p1 = indptr[b + 1];
    const int io0 = item_off[b], io1 = item_off[b + 1];
    if (hb != batch || hk != hkv) return;
    np = p1 - p0;
    nsplit = (io1 - io0) / hkv;
    i0 = io0 + kvh;
  }
  uint16_t* op = out + ((int64_t)b * hq + h) * D + lane * V;
  const int64_t gi = ((int64_t)b * hq + h) * ldg + lane * V;  // the gate row's columns (with a gate)
  if (np == 0) {
#pragma unroll
    for (int j = 0; j < V; ++j) op[j] = (uint16_t)gated_bf16(0.f, gate, gi + j);
    return;
  }
  if (nsplit <= 1) return;  // written by the decode kernel
  float mm = -INFINITY, ll = 0.f, acc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) acc[j] = 0.f;
  for (int c0 = 0; c0 < nsplit; c0 += P) {
    // item of split i: i0 + i hkv (items are in (split, KV head) order); clamped: in-bounds, weight zeroed below
    const int js = min(c0 + (lane & (P - 1)), nsplit - 1);
    const int64_t ij = (int64_t)(i0 + js * hkv) * group + hh;
    const float mj = part_m[ij], lj = part_l[ij];
    float oi[P][V];
#pragma unroll
    for (int k = 0; k < P; ++k) {
      const float* src = part_o + ((int64_t)(i0 + min(c0 + k, nsplit - 1) * hkv) * group + hh) * D + lane * V;
#pragma unroll
      for (int j = 0; j < V; ++j) oi[k][j] = src[j];
    }
    const bool jv = (lane < P) && (c0 + lane < nsplit) && mj != -INFINITY;
    const float cm = fmaxf(mm, wave_max(jv ? mj : -INFINITY));
    const float wj = jv ? exp2f(mj - cm) : 0.f;  // lane j < P: split c0 + j's weight
    const float sc = mm == -INFINITY ? 0.f : exp2f(mm - cm);
    ll = ll * sc + wave_sum(wj * lj);
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] *= sc;
#pragma unroll
    for (int k = 0; k < P; ++k) {
      const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wj), k));
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] += w * oi[k][j];
    }
    mm = cm;
  }
  const float inv = ll > 0.f ? 1.0f / ll : 0.f;
#pragma unroll
  for (int j = 0; j < V; ++j) op[j] = (uint16_t)gated_bf16(acc[j] * inv, gate, gi + j);
}

// cache[loc[b,0], 0, loc[b,1], kvh, :] = k[b, kvh, :]; plane 1 <- v (store_paged_kv, flash_attn.py:53-84).
__global__ __launch_bounds__(256) void paged_kv_write_kernel(const uint16_t* __restrict__ k,
                                                             const uint16_t* __restrict__ v,
                                                             uint16_t* __restrict__ cache,
                                                             const int* __restrict__ loc, int batch, int hkv,
                                                             int d, int page_size, int64_t num_pages,
                                                             int* __restrict__ status) {
  const int row_chunks = hkv * d / 8;  // 16-byte chunks of one token row
  const int64_t total = (int64_t)batch * row_chunks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2 * total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int plane = i >= total;
    const int64_t j = plane ? i - total : i;
    const int b = (int)(j / row_chunks), ch = (int)(j - (int64_t)b * row_chunks);
    const int page = loc[2 * b], off = loc[2 * b + 1];
    if (page < 0 || page >= num_pages || off < 0 || off >= page_size) {
      if (status) *status = 1;
      continue;
    }
    const uint16_t* src = (plane ? v : k) + (int64_t)b * hkv * d + ch * 8;
    uint16_t* dst = cache + (((int64_t)page * 2 + plane) * page_size + off) * (int64_t)hkv * d + ch * 8;
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  }
}

// The FP8 cache's KV write: cache[loc[b,0], plane, loc[b,1], kvh, :] = e4m3(bf16(x * scale)) for x = k (plane 0)
// and v (plane 1) (q35_group.py:244-247, KV8=2). One thread per 8 elements.
__global__ __launch_bounds__(256) void paged_kv_write_fp8_kernel(const uint16_t* __restrict__ k,
                                                                 const uint16_t* __restrict__ v,
                                                                 unsigned char* __restrict__ cache,
                                                                 const int* __restrict__ loc, int batch, int hkv,
                                                                 int d, int page_size, int64_t num_pages, float scale,
                                                                 int* __restrict__ status) {
  const int row_chunks = hkv * d / 8;
  const int64_t total = (int64_t)batch * row_chunks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2 * total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int plane = i >= total;
    const int64_t j = plane ? i - total : i;
    const int b = (int)(j / row_chunks), ch = (int)(j - (int64_t)b * row_chunks);
    const int page = loc[2 * b], off = loc[2 * b + 1];
    if (page < 0 || page >= num_pages || off < 0 || off >= page_size) {
      if (status) *status = 1;
      continue;
    }
    const uint4 src = *reinterpret_cast<const uint4*>((plane ? v : k) + (int64_t)b * hkv * d + ch * 8);
    const uint32_t w[4] = {src.x, src.y, src.z, src.w};
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = __uint_as_float(e & 1 ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
      const uint32_t c = f32_to_e4m3(round_bf16(x * scale));
      if (e < 4) lo |= c << (8 * e); else hi |= c << (8 * (e - 4));
    }
    unsigned char* dst = cache + (((int64_t)page * 2 + plane) * page_size + off) * (int64_t)hkv * d + ch * 8;
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
  }
}

// ---- Multi-token (prefill / verify) attention over the paged cache, causal ----
// The qlen new tokens of sequence b are the last qlen of its kv_len cached tokens (they are written before the call),
// so token t sits at position kv_len - qlen + t and sees cached tokens 0 .. that position (the causal bias of the
// current block, flash_attn.py:484-486; q35_prefill.py:264-300 masks the block the same way). The query rows of one
// (sequence, KV head) are r = t * G + h for the G query heads h of the KV head: a workgroup takes 128 consecutive
// rows (8 waves x 16) and streams the K / V tiles its rows can see, up to its last row's position, through a
// direct-to-LDS ring (the decode kernel's tile layout, loads issued by the first 4 waves). Each wave computes
// S^T = K Q^T for its 16 rows and O^T += V^T P^T over the whole head dim. 16 rows per wave keep Q and O in
// 100 VGPRs (two waves per SIMD); 32 rows per wave overflowed the VGPRs and the compiler moved O between AGPRs and
// VGPRs on every tile (measured: 700 VALU instructions per tile, 608 us for the 4096-token chunk).
typedef short axk_s16x8 __attribute__((ext_vector_type(8)));
constexpr int kPfWaves = 8;
constexpr int kPfRowsPerWave = 16;
constexpr int kPfNI = kPfRowsPerWave / 16;  // 16-row MFMA blocks per wave
constexpr int kPfRows = kPfWaves * kPfRowsPerWave;
constexpr int kPfAhead = 6;  // tiles in flight while two are computed (even: tiles are taken in pairs)
constexpr int kPfBuf = kPfAhead + 2;

template <int D>
__global__ __launch_bounds__(64 * kPfWaves) void paged_prefill_kernel(
    const uint16_t* __restrict__ q, const unsigned char* __restrict__ cache, const int* __restrict__ qo_indptr,
    const int* __restrict__ indptr, const int* __restrict__ last_page_len, const int* __restrict__ indices,
    int batch, int total_q, int hq, int hkv, int page_size, int64_t num_pages, float sm_scale, int xcd_per_head,
    int* __restrict__ status, uint16_t* __restrict__ out, const uint16_t* __restrict__ gate, int64_t ldg) {
  using C = PagedCfg<D>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int group = hq / hkv;
  // KV head and block index: consecutive workgroups go to the 8 XCDs in turn, so with xcd_per_head > 0 the blocks of
  // one KV head run on xcd_per_head XCDs only and its K / V stay in their L2s
  int kvh, want;
  if (xcd_per_head > 0) {
    const int x = blockIdx.x & 7, sl = blockIdx.x >> 3;
    kvh = x / xcd_per_head;
    want = sl * xcd_per_head + (x - kvh * xcd_per_head);
  } else {
    kvh = blockIdx.x % hkv;
    want = blockIdx.x / hkv;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;

  // this workgroup's (sequence, row block): the blocks of each sequence in turn, its last (longest) block first.
  // Every wave derives the same answer; the grid is an upper bound and surplus workgroups return.
  int b = -1, blk = 0;
  for (int c0 = 0, base = 0; c0 < batch && b < 0; c0 += 64) {
    const int sq = c0 + lane;
    const int qlen_l = sq < batch ? qo_indptr[sq + 1] - qo_indptr[sq] : 0;
    const int nb = qlen_l > 0 ? (qlen_l * group + kPfRows - 1) / kPfRows : 0;
    int incl = nb;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    const int excl = base + incl - nb;
    const unsigned long long hit = __builtin_amdgcn_ballot_w64(nb > 0 && want >= excl && want < excl + nb);
    if (hit) {
      const int hl = __builtin_ctzll(hit);
      b = c0 + hl;
      blk = __shfl(nb, hl, 64) - 1 - (want - __shfl(excl, hl, 64));
    }
    base += __shfl(incl, 63, 64);
  }
  if (b < 0) return;
  const int q0 = qo_indptr[b], qlen = qo_indptr[b + 1] - q0;
  if (q0 < 0 || q0 + qlen > total_q) {  // a query range outside q: nothing is read or written
    if (status && threadIdx.x == 0) *status = 1;
    return;
  }
  const int pb = indptr[b], npg = max(indptr[b + 1] - pb, 0);
  const int last = min(max(npg > 0 ? last_page_len[b] : 0, 0), page_size);
  const int kv_len = npg > 0 ? (npg - 1) * page_size + last : 0;
  const int tpp = page_size / kTile;
  const int r_first = blk * kPfRows, r_last = min(r_first + kPfRows, qlen * group) - 1;
  const int base_pos = kv_len - qlen;  // position of new token 0 (negative if the cache lacks the new tokens)
  const int kv_end = min(kv_len, max(0, base_pos + r_last / group + 1));
  const int ntiles = min((kv_end + kTile - 1) / kTile, npg * tpp);
  const float c = sm_scale * kLog2e;
  const int64_t row_stride = (int64_t)hkv * D * 2, plane_stride = (int64_t)page_size * row_stride;
  const uint32_t lds0 = lds_addr(smem);

  // rows of this wave: block i holds row r_first + kPfRowsPerWave wave + 16 i + l16 (replicated over g)
  int pos[kPfNI];
  int64_t qoff[kPfNI];
  axk_bf16x8 qb[kPfNI][C::KSTEPS];
#pragma unroll
  for (int i = 0; i < kPfNI; ++i) {
    const int r = r_first + kPfRowsPerWave * wave + 16 * i + l16;
    const bool valid = r <= r_last;
    const int t = valid ? r / group : 0, h = valid ? r - t * group : 0;
    pos[i] = valid ? base_pos + t : -1;
    qoff[i] = ((int64_t)(q0 + t) * hq + kvh * group + h) * D;
    const uint16_t* qp = q + qoff[i] + 8 * g;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) qb[i][s] = valid ? load_bf16x8(qp + 32 * s) : zero_bf16x8();
  }
  int chunk = 0;
  int pid = lane < npg ? indices[pb + lane] : 0;
  asm volatile("" : "+v"(pid));
#pragma unroll
  for (int i = 0; i < kPfNI; ++i)
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) asm volatile("" : "+v"(qb[i][s]));

  auto locate = [&](int ti, int& nvalid) -> const unsigned char* {
    const int lp = ti / tpp, tp = ti - lp * tpp;
    if ((lp >> 6) != chunk) {
      chunk = lp >> 6;
      const int j = (chunk << 6) + lane;
      pid = j < npg ? indices[pb + j] : 0;
      asm volatile("" : "+v"(pid));
    }
    int page = __builtin_amdgcn_readlane(pid, lp & 63);  // lp is wave-uniform: a lane read, no LDS round trip
    const int valid_in_page = (lp == npg - 1) ? last : page_size;
    nvalid = min(kTile, valid_in_page - tp * kTile);
    if (page < 0 || page >= num_pages) {
      if (status && lane == 0 && nvalid > 0) *status = 1;
      page = 0;
      nvalid = 0;
    }
    return cache + (int64_t)page * 2 * plane_stride + (int64_t)(tp * kTile) * row_stride + (int64_t)kvh * D * 2;
  };
  int lane_tok[C::IPW];
  int64_t lane_off[C::IPW], lane_off0[C::IPW];
#pragma unroll
  for (int k = 0; k < C::IPW; ++k) {
    const int j = wave * C::IPW + k;
    const int plane = j / C::IPP, blk2 = j - plane * C::IPP;
    lane_tok[k] = blk2 * C::RPI + lane / (C::RB / 16);
    lane_off0[k] = plane * plane_stride + (lane % (C::RB / 16)) * 16;
    lane_off[k] = lane_off0[k] + (int64_t)lane_tok[k] * row_stride;
  }
  auto issue = [&](int ti, int nb) -> int {
    int nvalid;
    const unsigned char* kbase = locate(ti < ntiles ? ti : ntiles - 1, nvalid);
    const int nrow = nvalid > 0 ? nvalid : 1;
    if (wave < kWaves)  // wave-uniform: the first four waves load the tile
#pragma unroll
    for (int k = 0; k < C::IPW; ++k) {
      const int j = wave * C::IPW + k;
      const int plane = j / C::IPP, blk2 = j - plane * C::IPP;
      lds_dma16(kbase + (lane_tok[k] < nrow ? lane_off[k] : lane_off0[k]),
                lds0 + nb * C::BUF + plane * C::PLANE + blk2 * C::BLK);
    }
    return ti < ntiles ? nvalid : 0;
  };

  constexpr int DT = D / 16;
  axk_f32x4 o[kPfNI][DT];
  float m_run[kPfNI], l_run[kPfNI];
#pragma unroll
  for (int i = 0; i < kPfNI; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
#pragma unroll
    for (int t = 0; t < DT; ++t) o[i][t] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // the math of tiles ti and ti + 1 (K planes ka, kb; V planes PLANE after them; na, nb valid tokens). The 32 tokens
  // are one k-step of the 16x16x32 PV MFMA: k = 8 g + j is token 4 g + j of tile ti for j < 4 and token 4 g + j - 4
  // of tile ti + 1 otherwise, in both operands (P^T from the two score tiles, V^T from one transposing read of each).
  // The softmax reference max is raised only when a row's scores pass it by more than kPfSlack (log2 units), so
  // p <= 2^kPfSlack and O is rescaled only on those rare tiles.
  constexpr float kPfSlack = 8.0f;
  // the lowest position among this wave's rows (-1 if it holds an invalid row): a pair of full tiles wholly at or
  // before it needs no mask (every wave-uniform)
  int pos_lo = pos[0];
#pragma unroll
  for (int i = 1; i < kPfNI; ++i) pos_lo = min(pos_lo, pos[i]);
#pragma unroll
  for (int o2 = 1; o2 < 16; o2 <<= 1) pos_lo = min(pos_lo, __shfl_xor(pos_lo, o2, 64));
  auto pair_math = [&](const unsigned char* ka, const unsigned char* kb, int ti, int na, int nb, bool full) {
    axk_f32x4 sa[kPfNI], sb[kPfNI];
#pragma unroll
    for (int i = 0; i < kPfNI; ++i) sa[i] = sb[i] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
    const int roff = C::row_off(l16) + 16 * g;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) {
      const axk_bf16x8 fa = *reinterpret_cast<const axk_bf16x8*>(ka + roff + 64 * s);
      const axk_bf16x8 fb = *reinterpret_cast<const axk_bf16x8*>(kb + roff + 64 * s);
#pragma unroll
      for (int i = 0; i < kPfNI; ++i) {
        sa[i] = mfma_bf16_16x16x32(fa, qb[i][s], sa[i]);
        sb[i] = mfma_bf16_16x16x32(fb, qb[i][s], sb[i]);
      }
    }
    const int tok0 = ti * kTile + 4 * g;
    axk_bf16x8 pb8[kPfNI];
    float alpha[kPfNI];
    bool moved = false;
#pragma unroll
    for (int i = 0; i < kPfNI; ++i) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        sa[i][rr] *= c;
        sb[i][rr] *= c;
      }
      if (!full) {
        // token tok0 + rr of tile ti is visible iff rr <= la (inside the tile's valid rows and at or before the
        // row's position); tile ti + 1 likewise with lb
        const int la = min(pos[i], ti * kTile + na - 1) - tok0;
        const int lb = min(pos[i], ti * kTile + kTile + nb - 1) - tok0 - kTile;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          if (rr > la) sa[i][rr] = -INFINITY;
          if (rr > lb) sb[i][rr] = -INFINITY;
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) mx = fmaxf(mx, fmaxf(sa[i][rr], sb[i][rr]));
      mx = xor32_max(xor16_max(mx));
      const bool raise = mx > m_run[i] + kPfSlack;  // -inf + slack stays -inf: a row's first visible score raises
      moved |= __builtin_amdgcn_ballot_w64(raise) != 0;
      alpha[i] = raise ? __builtin_amdgcn_exp2f(m_run[i] - mx) : 1.0f;
      if (raise) m_run[i] = mx;
      // a row that has seen nothing stays at zero: its scores are all -inf and exp2(-inf) = 0
      const float m_use = m_run[i] == -INFINITY ? 0.f : m_run[i];
      axk_s16x8 pbits;
      float psum = 0.f;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float pa = __builtin_amdgcn_exp2f(sa[i][rr] - m_use);
        const float pbv = __builtin_amdgcn_exp2f(sb[i][rr] - m_use);
        psum += pa + pbv;
        pbits[rr] = (short)f32_to_bf16_bits(pa);
        pbits[4 + rr] = (short)f32_to_bf16_bits(pbv);
      }
      pb8[i] = __builtin_bit_cast(axk_bf16x8, pbits);
      psum = xor32_sum(xor16_sum(psum));
      l_run[i] = l_run[i] * alpha[i] + psum;
    }
    if (moved) {  // wave-uniform and rare: a branch, not a select per accumulator
#pragma unroll
      for (int i = 0; i < kPfNI; ++i)
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) o[i][t][rr] *= alpha[i];
    }
    const int voff = C::PLANE + C::row_off(4 * g + (l16 >> 2)) + 8 * (l16 & 3);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const axk_s16x4 va = lds_read_tr16(ka + voff + 32 * t);
      const axk_s16x4 vb = lds_read_tr16(kb + voff + 32 * t);
      const axk_bf16x8 v8 = __builtin_bit_cast(axk_bf16x8, __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int i = 0; i < kPfNI; ++i) o[i][t] = mfma_bf16_16x16x32(v8, pb8[i], o[i][t]);
    }
  };

  if (ntiles > 0) {
    // tiles land kPfAhead ahead in a ring of kPfBuf = kPfAhead + 2; an iteration computes two
    int nv[kPfAhead];  // valid tokens of tiles ti .. ti + kPfAhead - 1
#pragma unroll
    for (int j = 0; j < kPfAhead; ++j) nv[j] = issue(j, j);
    for (int ti = 0; ti < ntiles; ti += 2) {
      wait_vmcnt<(kPfAhead - 2) * C::IPW>();  // this wave's loads of tiles ti, ti + 1 have landed
      __builtin_amdgcn_s_barrier();            // ... and every wave's; all are done with tiles ti - 2, ti - 1
      const int n0 = issue(ti + kPfAhead, (ti + kPfAhead) % kPfBuf);  // into the buffers of tiles ti - 2, ti - 1
      const int n1 = issue(ti + kPfAhead + 1, (ti + kPfAhead + 1) % kPfBuf);
      const int na = nv[0], nb = nv[1];
#pragma unroll
      for (int j = 0; j + 2 < kPfAhead; ++j) nv[j] = nv[j + 2];
      nv[kPfAhead - 2] = n0;
      nv[kPfAhead - 1] = n1;
      unsigned char* ka = smem + (ti % kPfBuf) * C::BUF;
      unsigned char* kb = smem + ((ti + 1) % kPfBuf) * C::BUF;
      const bool full = na == kTile && nb == kTile && ti * kTile + 2 * kTile - 1 <= pos_lo;
      if (na + nb > 0) pair_math(ka, kb, ti, na, nb, full);
    }
    wait_vmcnt<0>();
  }

  // lane (row l16 of block i, g) holds O[row][d = 16 t + 4 g .. + 3]
#pragma unroll
  for (int i = 0; i < kPfNI; ++i) {
    const int r = r_first + kPfRowsPerWave * wave + 16 * i + l16;
    if (r > r_last) continue;
    const float inv = l_run[i] > 0.f ? 1.0f / l_run[i] : 0.f;
    const int64_t gi0 = qoff[i] / D * ldg;  // the row's gate (with a gate)
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int col = 16 * t + 4 * g;
      uint2 w;
      w.x = gated_bf16(o[i][t][0] * inv, gate, gi0 + col) | (gated_bf16(o[i][t][1] * inv, gate, gi0 + col + 1) << 16);
      w.y = gated_bf16(o[i][t][2] * inv, gate, gi0 + col + 2) | (gated_bf16(o[i][t][3] * inv, gate, gi0 + col + 3) << 16);
      *reinterpret_cast<uint2*>(out + qoff[i] + col) = w;
    }
  }
}

template <int D>
int launch_prefill(const uint16_t* q, const void* cache, const int* qo_indptr, const int* indptr, const int* last,
                   const int* indices, uint16_t* out, int batch, int total_q, int hq, int hkv, int page_size,
                   int64_t num_pages, float sm_scale, int* status, hipStream_t st, const uint16_t* gate = nullptr,
                   int64_t ldg = 0) {
  const int64_t rows = (int64_t)total_q * (hq / hkv);
  const int64_t nblk = (rows + kPfRows - 1) / kPfRows + batch;  // >= the sum over sequences of their row blocks
  const int xph = hkv <= 8 && 8 % hkv == 0 ? 8 / hkv : 0;      // XCDs per KV head
  const int64_t grid = xph ? 8 * ((nblk + xph - 1) / xph) : nblk * hkv;
  if (grid > 0x7fffffff) return AXK_E_SHAPE;
  const size_t lds = (size_t)kPfBuf * PagedCfg<D>::BUF;
  static AxkOnce lds_once;  // > 64 KiB of dynamic LDS must be allowed once per kernel
  if (const int rc = axk_raise_lds(lds_once, reinterpret_cast<const void*>(&paged_prefill_kernel<D>), lds)) return rc;
  AXK_LAUNCH_GATE();
  hipLaunchKernelGGL((paged_prefill_kernel<D>), dim3((unsigned)grid), dim3(64 * kPfWaves), lds, st, q,
                     static_cast<const unsigned char*>(cache), qo_indptr, indptr, last, indices, batch, total_q, hq,
                     hkv, page_size, num_pages, sm_scale, xph, status, out, gate, ldg);
  return axk_launch_status();
}

struct WsView {
  PlanHeader* hdr;
  int* item_off;
  ItemDesc* descs;
  float *pm, *pl, *po;
};

WsView ws_view(void* ws, int batch, int hkv, int group, int d) {
  size_t oi, od, om, ol, oo;
  ws_layout(batch, hkv, group, d, &oi, &od, &om, &ol, &oo);
  unsigned char* w = reinterpret_cast<unsigned char*>(ws);
  return {reinterpret_cast<PlanHeader*>(w), reinterpret_cast<int*>(w + oi), reinterpret_cast<ItemDesc*>(w + od),
          reinterpret_cast<float*>(w + om), reinterpret_cast<float*>(w + ol), reinterpret_cast<float*>(w + oo)};
}

// Split workgroups per CU (and the plan's slot count per CU). Two, not the three that LDS would allow: fewer,
// larger items carry fewer per-item prologues and fp32 partials (measured, config 1: 55.7 us with three per CU,
// 51.7 us with two, 73.8 us with one).
constexpr int kBlocksPerCU = 2;

// Compute units of the current device (cached per device).
int device_cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

// Workgroups of the split kernel (also the slot count the local plan divides the work by).
int split_grid(int batch, int hkv) {
  const unsigned items = (unsigned)ws_items_max(batch, hkv);
  const unsigned slots = (unsigned)(kBlocksPerCU * device_cu_count());
  return (int)(items < slots ? items : slots);
}

// The split kernel's dynamic LDS: a bf16 cache: the ring of tile pairs; an 8-bit cache: the waves' V slots (the
// end-of-item merge reuses them).
template <int D, int KB, int QM>
constexpr size_t split_lds() {
  return KB == 1 ? (size_t)WaveCfg<D>::LDS : (size_t)kNBufPair * PagedCfg<D>::BUF;
}

// Allows the split kernel its dynamic LDS (above 64 KiB), once per process.
template <int D, int KB, int QM>
int raise_split_lds() {
  static AxkOnce once;
  return axk_raise_lds(once, reinterpret_cast<const void*>(&paged_decode_kernel<D, KB, QM>), split_lds<D, KB, QM>());
}

template <int D, int KB = 2, int QM = 0>
int launch_split(const uint16_t* q, const void* cache, const int* indptr, const int* last, const int* indices,
                 uint16_t* out, int batch, int hq, int hkv, int page_size, int64_t num_pages, float sm_scale,
                 void* ws, hipStream_t st, float inv_scale = 1.0f, int bias = 0, const void* kv_scales = nullptr,
                 const uint16_t* gate = nullptr, int64_t ldg = 0) {
  const int group = hq / hkv;
  const WsView v = ws_view(ws, batch, hkv, group, D);
  // the kernel's per-lane tile offsets are 32-bit: both planes of a page stay under 2^31 bytes
  AXK_REQUIRE((int64_t)2 * page_size * hkv * D * KB < ((int64_t)1 << 31), AXK_E_SHAPE);
  constexpr size_t lds = split_lds<D, KB, QM>();
  if (const int rc = raise_split_lds<D, KB, QM>()) return rc;
  const int local = batch <= kLocalPlanBatch ? 1 : 0;
  hipLaunchKernelGGL((paged_decode_kernel<D, KB, QM>), dim3((unsigned)split_grid(batch, hkv)), dim3(64 * kWaves),
                     lds, st, q, static_cast<const unsigned char*>(cache), indptr, last, indices, batch, hq, hkv,
                     page_size, num_pages, sm_scale, inv_scale, static_cast<const unsigned char*>(kv_scales), local,
                     bias, v.hdr, v.descs, v.pm, v.pl, v.po, out, gate, ldg);
  return axk_launch_status();
}

template <int D>
int launch_merge(const int* indptr, const int* last, uint16_t* out, int batch, int hq, int hkv, int page_size,
                 void* ws, hipStream_t st, int kb = 2, int bias = 0, const uint16_t* gate = nullptr, int64_t ldg = 0) {
  const WsView v = ws_view(ws, batch, hkv, hq / hkv, D);
  const int local = batch <= kLocalPlanBatch ? 1 : 0;
  hipLaunchKernelGGL((paged_merge_kernel<D>), dim3((unsigned)((batch * hq + 3) / 4)), dim3(256), 0, st, indptr, last,
                     v.hdr,
                     v.item_off, batch, hq, hkv, split_grid(batch, hkv), local, bias, v.pm, v.pl, v.po, out, gate, ldg);
  return axk_launch_status();
}

int check_heads(int64_t batch, int64_t hq, int64_t hkv, int64_t d) {
  AXK_REQUIRE(batch > 0 && batch <= (1 << 20) && hkv > 0 && hq > 0, AXK_E_SHAPE);
  AXK_REQUIRE(hq % hkv == 0 && hq / hkv <= kMaxGroup, AXK_E_SHAPE);
  AXK_REQUIRE(d == 64 || d == 128 || d == 256, AXK_E_SHAPE);
  return AXK_OK;
}

}  // namespace

extern "C" size_t axk_paged_decode_workspace_size(int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                                  int64_t head_dim) {
  if (check_heads(batch, num_qo_heads, num_kv_heads, head_dim) != AXK_OK) return 0;
  size_t a, b, c, d, e;
  return ws_layout(batch, num_kv_heads, num_qo_heads / num_kv_heads, head_dim, &a, &b, &c, &d, &e);
}

namespace {

int check_page(int64_t page_size) {
  return page_size >= kTile && page_size % kTile == 0 && page_size <= 4096 ? AXK_OK : AXK_E_SHAPE;
}

int check_ws(void* workspace, size_t workspace_bytes, int64_t batch, int64_t hq, int64_t hkv, int64_t d) {
  const size_t need = axk_paged_decode_workspace_size(batch, hq, hkv, d);
  return workspace && workspace_bytes >= need && axk_aligned(workspace, 256) ? AXK_OK : AXK_E_WORKSPACE;
}

// The plan (launched only above kLocalPlanBatch sequences). bias: 0 when last_page_len counts the valid tokens of
// the last page, 1 when it counts the history only and the current token (written at the next slot) is attended too.
int decode_plan(const int32_t* indptr, const int32_t* last_page_len, int64_t batch, int64_t hq, int64_t hkv,
                int64_t d, int64_t page_size, int kb, int bias, void* workspace, size_t workspace_bytes,
                hipStream_t st) {
  AXK_REQUIRE(indptr && last_page_len, AXK_E_NULL);
  int rc = check_heads(batch, hq, hkv, d);
  if (rc != AXK_OK) return rc;
  if ((rc = check_page(page_size)) != AXK_OK) return rc;
  if ((rc = check_ws(workspace, workspace_bytes, batch, hq, hkv, d)) != AXK_OK) return rc;
  if (batch <= kLocalPlanBatch) return AXK_OK;  // the split and merge kernels derive their partition themselves
  (void)kb;
  AXK_LAUNCH_GATE();
  const WsView v = ws_view(workspace, (int)batch, (int)hkv, (int)(hq / hkv), (int)d);
  hipLaunchKernelGGL(paged_plan_kernel, dim3(1), dim3(256), 0, st, indptr, last_page_len, bias, (int)batch, (int)hkv,
                     (int)page_size, kBlocksPerCU * device_cu_count(), v.hdr, v.item_off, v.descs);
  return axk_launch_status();
}

// Every check of the split (and of the merge that follows it) on the host, before anything is launched.
int check_split(const void* q, const void* kv_cache, const int32_t* indptr, const int32_t* indices,
                const int32_t* last_page_len, const void* out, int64_t batch, int64_t hq, int64_t hkv, int64_t d,
                int64_t page_size, int64_t num_pages, void* workspace, size_t workspace_bytes) {
  AXK_REQUIRE(q && kv_cache && indptr && indices && last_page_len && out, AXK_E_NULL);
  int rc = check_heads(batch, hq, hkv, d);
  if (rc != AXK_OK) return rc;
  if ((rc = check_page(page_size)) != AXK_OK) return rc;
  AXK_REQUIRE(num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(q, 16) && axk_aligned(kv_cache, 16), AXK_E_ALIGN);
  if ((rc = check_ws(workspace, workspace_bytes, batch, hq, hkv, d)) != AXK_OK) return rc;
  const size_t qbytes = (size_t)batch * hq * d * 2;
  AXK_REQUIRE(!axk_overlap(out, qbytes, q, qbytes), AXK_E_ALIAS);
  AXK_REQUIRE(!axk_overlap(out, qbytes, workspace, workspace_bytes), AXK_E_ALIAS);
  return AXK_OK;
}

int decode_split(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
                 const int32_t* last_page_len, uint16_t* out, int64_t batch, int64_t hq, int64_t hkv, int64_t d,
                 int64_t page_size, int64_t num_pages, float sm_scale, int bias, void* workspace,
                 hipStream_t st, const uint16_t* gate = nullptr, int64_t ldg = 0) {
  const int B = (int)batch, HQ = (int)hq, HKV = (int)hkv, PS = (int)page_size;
  switch (d) {
    case 64:
      return launch_split<64>(q, kv_cache, indptr, last_page_len, indices, out, B, HQ, HKV, PS, num_pages, sm_scale,
                              workspace, st, 1.0f, bias, nullptr, gate, ldg);
    case 128:
      return launch_split<128>(q, kv_cache, indptr, last_page_len, indices, out, B, HQ, HKV, PS, num_pages, sm_scale,
                               workspace, st, 1.0f, bias, nullptr, gate, ldg);
    default:
      return launch_split<256>(q, kv_cache, indptr, last_page_len, indices, out, B, HQ, HKV, PS, num_pages, sm_scale,
                               workspace, st, 1.0f, bias, nullptr, gate, ldg);
  }
}

int decode_merge(const int32_t* indptr, const int32_t* last_page_len, uint16_t* out, int64_t batch, int64_t hq,
                 int64_t hkv, int64_t d, int64_t page_size, int kb, int bias, void* workspace, hipStream_t st,
                 const uint16_t* gate = nullptr, int64_t ldg = 0) {
  const int B = (int)batch, HQ = (int)hq, HKV = (int)hkv, PS = (int)page_size;
  switch (d) {
    case 64: return launch_merge<64>(indptr, last_page_len, out, B, HQ, HKV, PS, workspace, st, kb, bias, gate, ldg);
    case 128: return launch_merge<128>(indptr, last_page_len, out, B, HQ, HKV, PS, workspace, st, kb, bias, gate, ldg);
    default: return launch_merge<256>(indptr, last_page_len, out, B, HQ, HKV, PS, workspace, st, kb, bias, gate, ldg);
  }
}

// plan + split + merge of the bf16 cache, every check first
int decode_all(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
               const int32_t* last_page_len, uint16_t* out, int64_t batch, int64_t hq, int64_t hkv, int64_t d,
               int64_t page_size, int64_t num_pages, float sm_scale, int bias, void* workspace, size_t workspace_bytes,
               hipStream_t st, const uint16_t* gate = nullptr, int64_t ldg = 0) {
  int rc = check_split(q, kv_cache, indptr, indices, last_page_len, out, batch, hq, hkv, d, page_size, num_pages,
                       workspace, workspace_bytes);
  if (rc != AXK_OK) return rc;
  if ((rc = decode_plan(indptr, last_page_len, batch, hq, hkv, d, page_size, 2, bias, workspace, workspace_bytes,
                        st)) != AXK_OK)
    return rc;
  AXK_LAUNCH_GATE();
  if ((rc = decode_split(q, kv_cache, indptr, indices, last_page_len, out, batch, hq, hkv, d, page_size, num_pages,
                         sm_scale, bias, workspace, st, gate, ldg)) != AXK_OK)
    return rc;
  return decode_merge(indptr, last_page_len, out, batch, hq, hkv, d, page_size, 2, bias, workspace, st, gate, ldg);
}

}  // namespace

extern "C" int axk_paged_decode_plan(const int32_t* indptr, const int32_t* last_page_len, int64_t batch,
                                     int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                     void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  return decode_plan(indptr, last_page_len, batch, num_qo_heads, num_kv_heads, head_dim, page_size, 2, 0, workspace,
                     workspace_bytes, axk_stream(stream));
}

extern "C" int axk_paged_decode_split(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                                      const int32_t* indices, const int32_t* last_page_len, uint16_t* out,
                                      int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                      int64_t page_size, int64_t num_pages, float sm_scale, void* workspace,
                                      size_t workspace_bytes, axk_stream_t stream) {
  const int rc = check_split(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads,
                             head_dim, page_size, num_pages, workspace, workspace_bytes);
  if (rc != AXK_OK) return rc;
  return decode_split(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim,
                      page_size, num_pages, sm_scale, 0, workspace, axk_stream(stream));
}

extern "C" int axk_paged_decode_merge(const int32_t* indptr, const int32_t* last_page_len, uint16_t* out,
                                      int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                      int64_t page_size, void* workspace, size_t workspace_bytes,
                                      axk_stream_t stream) {
  AXK_REQUIRE(indptr && last_page_len && out, AXK_E_NULL);
  int rc = check_heads(batch, num_qo_heads, num_kv_heads, head_dim);
  if (rc != AXK_OK) return rc;
  if ((rc = check_page(page_size)) != AXK_OK) return rc;
  if ((rc = check_ws(workspace, workspace_bytes, batch, num_qo_heads, num_kv_heads, head_dim)) != AXK_OK) return rc;
  return decode_merge(indptr, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim, page_size, 2, 0,
                      workspace, axk_stream(stream));
}

extern "C" int axk_paged_decode_run(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                                    const int32_t* indices, const int32_t* last_page_len, uint16_t* out,
                                    int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                    int64_t page_size, int64_t num_pages, float sm_scale, void* workspace,
                                    size_t workspace_bytes, axk_stream_t stream) {
  const int rc = check_split(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads,
                             head_dim, page_size, num_pages, workspace, workspace_bytes);
  if (rc != AXK_OK) return rc;
  hipStream_t st = axk_stream(stream);
  const int rs = decode_split(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads,
                              head_dim, page_size, num_pages, sm_scale, 0, workspace, st);
  if (rs != AXK_OK) return rs;
  return decode_merge(indptr, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim, page_size, 2, 0,
                      workspace, st);
}

extern "C" int axk_paged_decode(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                                const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                                int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                int64_t num_pages, float sm_scale, void* workspace, size_t workspace_bytes,
                                axk_stream_t stream) {
  return decode_all(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim,
                    page_size, num_pages, sm_scale, 0, workspace, workspace_bytes, axk_stream(stream));
}

int axk_paged_decode_gated(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
                           const int32_t* last_page_len, const uint16_t* gate, int64_t ldg, uint16_t* out,
                           int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                           int64_t page_size, int64_t num_pages, float sm_scale, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  AXK_REQUIRE(gate, AXK_E_NULL);
  AXK_REQUIRE(ldg >= head_dim, AXK_E_SHAPE);
  const size_t gbytes = (size_t)((batch * num_qo_heads - 1) * ldg + head_dim) * 2;
  AXK_REQUIRE(!axk_overlap(out, (size_t)batch * num_qo_heads * head_dim * 2, gate, gbytes), AXK_E_ALIAS);
  return decode_all(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim,
                    page_size, num_pages, sm_scale, 0, workspace, workspace_bytes, stream, gate, ldg);
}

// ---- No-allocation variant: the workspace is a static device array of the library ----
namespace {
// The split partials of axk_paged_decode_noalloc. Host code never uses this name as an address: each device's copy
// is resolved once with hipGetSymbolAddress (scratch_ptr) and only that pointer is passed to kernels.
static __device__ __align__(256) unsigned char scratch[AXK_PAGED_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {nullptr};

// This device's copy of `scratch` (the current device), or nullptr if its address cannot be resolved.
void* scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}
}  // namespace

extern "C" int axk_paged_decode_noalloc(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                                        const int32_t* indices, const int32_t* last_page_len, uint16_t* out,
                                        int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                        int64_t page_size, int64_t num_pages, float sm_scale, axk_stream_t stream) {
  int rc = check_heads(batch, num_qo_heads, num_kv_heads, head_dim);
  if (rc != AXK_OK) return rc;
  const size_t need = axk_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim);
  AXK_REQUIRE(need <= AXK_PAGED_NOALLOC_SCRATCH_BYTES, AXK_E_SCRATCH);
  // The one-time set-up (this device's scratch address, the split kernel's LDS limit) is host work that must not
  // happen inside a stream capture: a first call on a device while its stream is capturing returns AXK_E_LAUNCH and
  // enqueues nothing (make one eager call first).
  {
    int dev = -1;
    bool ready = hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices;
    if (ready) {
      std::lock_guard<std::mutex> lock(g_scratch_mu);
      ready = g_scratch[dev] != nullptr;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    AXK_REQUIRE(hipStreamIsCapturing(axk_stream(stream), &cs) == hipSuccess, AXK_E_LAUNCH);
    AXK_REQUIRE(ready || cs == hipStreamCaptureStatusNone, AXK_E_LAUNCH);
  }
  void* ws = scratch_ptr();
  AXK_REQUIRE(ws, AXK_E_LAUNCH);
  switch (head_dim) {  // the split kernel's LDS limit, raised here (outside any capture) rather than at its launch
    case 64: rc = raise_split_lds<64, 2, 0>(); break;
    case 128: rc = raise_split_lds<128, 2, 0>(); break;
    default: rc = raise_split_lds<256, 2, 0>(); break;
  }
  if (rc != AXK_OK) return rc;
  return decode_all(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim,
                    page_size, num_pages, sm_scale, 0, ws, AXK_PAGED_NOALLOC_SCRATCH_BYTES, axk_stream(stream));
}

extern "C" int axk_paged_attention_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* kv_cache,
                                          const int32_t* indptr, const int32_t* indices,
                                          const int32_t* last_page_len, const int32_t* cache_location, uint16_t* out,
                                          int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                          int64_t head_dim, int64_t page_size, int64_t num_pages, float sm_scale,
                                          int32_t* status, void* workspace, size_t workspace_bytes,
                                          axk_stream_t stream) {
  AXK_REQUIRE(k && v && cache_location, AXK_E_NULL);
  AXK_REQUIRE(axk_aligned(k, 16) && axk_aligned(v, 16), AXK_E_ALIGN);
  int rc = check_split(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim,
                       page_size, num_pages, workspace, workspace_bytes);
  if (rc != AXK_OK) return rc;
  hipStream_t st = axk_stream(stream);
  const int64_t chunks = 2 * batch * num_kv_heads * head_dim / 8;
  const int64_t grid = chunks / 256 + 1 < 4096 ? chunks / 256 + 1 : 4096;
  AXK_LAUNCH_GATE();
  hipLaunchKernelGGL(paged_kv_write_kernel, dim3((unsigned)grid), dim3(256), 0, st, k, v, kv_cache, cache_location,
                     (int)batch, (int)num_kv_heads, (int)head_dim, (int)page_size, num_pages, status);
  if ((rc = axk_launch_status()) != AXK_OK) return rc;
  return decode_all(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim,
                    page_size, num_pages, sm_scale, 1, workspace, workspace_bytes, st);
}

extern "C" int axk_paged_kv_write(const uint16_t* k, const uint16_t* v, uint16_t* kv_cache,
                                  const int32_t* cache_location, int64_t batch, int64_t num_kv_heads,
                                  int64_t head_dim, int64_t page_size, int64_t num_pages, int32_t* status,
                                  axk_stream_t stream) {
  AXK_REQUIRE(k && v && kv_cache && cache_location, AXK_E_NULL);
  AXK_REQUIRE(batch >= 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 8 == 0, AXK_E_SHAPE);
  AXK_REQUIRE(page_size > 0 && num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(k, 16) && axk_aligned(v, 16) && axk_aligned(kv_cache, 16), AXK_E_ALIGN);
  if (batch == 0) return AXK_OK;
  const int64_t chunks = 2 * batch * num_kv_heads * head_dim / 8;
  int64_t grid = (chunks + 255) / 256;
  if (grid > 4096) grid = 4096;
  AXK_LAUNCH_GATE();
  hipLaunchKernelGGL(paged_kv_write_kernel, dim3((unsigned)grid), dim3(256), 0, axk_stream(stream), k, v, kv_cache,
                     cache_location, (int)batch, (int)num_kv_heads, (int)head_dim, (int)page_size, num_pages, status);
  return axk_launch_status();
}

namespace {
// The INT8 cache's KV write (q35_group.py kv_quant_row 197-205, kv_write_paged 250-255, KV8=1): per row and KV head
// s = bf16(max(amax, bf16(1e-5)) * bf16(1 / 127)), codes int8(bf16(x * bf16(1 / s))) rounded to nearest even and
// saturated, into cache[page, plane, slot, kvh, :]; s into scales[page, plane, slot, kvh]. Sixteen lanes per
// (token, plane, KV head) row, D / 16 values each; the row's amax by shuffles within the 16 lanes.
template <int D>
__global__ __launch_bounds__(256) void paged_kv_write_i8_kernel(const uint16_t* __restrict__ k,
                                                                const uint16_t* __restrict__ v,
                                                                unsigned char* __restrict__ cache,
                                                                uint16_t* __restrict__ scales,
                                                                const int* __restrict__ loc, int batch, int hkv,
                                                                int page_size, int64_t num_pages,
                                                                int* __restrict__ status) {
  constexpr int E = D / 16;  // values per lane (8 or 16)
  const int64_t rows = (int64_t)batch * 2 * hkv;
  const int sub = threadIdx.x & 15;
  for (int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4; row < rows;
       row += ((int64_t)gridDim.x * blockDim.x) >> 4) {
    const int b = (int)(row / (2 * hkv)), rem = (int)(row - (int64_t)b * 2 * hkv);
    const int plane = rem / hkv, kvh = rem - plane * hkv;
    const int page = loc[2 * b], off = loc[2 * b + 1];
    const bool bad = page < 0 || page >= num_pages || off < 0 || off >= page_size;  // uniform over the 16 lanes
    if (bad) {
      if (status && sub == 0) *status = 1;
      continue;
    }
    const uint16_t* src = (plane ? v : k) + ((int64_t)b * hkv + kvh) * D + sub * E;
    float x[E];
#pragma unroll
    for (int u = 0; u < E / 8; ++u) {
      const uint4 w = *reinterpret_cast<const uint4*>(src + 8 * u);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[8 * u + e] = __uint_as_float(e & 1 ? (ww[e >> 1] & 0xffff0000u) : (ww[e >> 1] << 16));
    }
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(x[e]));
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 16));
    const float kFloor = __uint_as_float(0x3728u << 16);    // bf16(1e-5)
    const float kInv127 = __uint_as_float(0x3c01u << 16);   // bf16(1 / 127)
    const float s = round_bf16(fmaxf(amax, kFloor) * kInv127);
    const float r = round_bf16(1.0f / s);
    uint32_t codes[E / 4];
#pragma unroll
    for (int c4 = 0; c4 < E / 4; ++c4) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y = fminf(fmaxf(rintf(round_bf16(x[4 * c4 + e] * r)), -128.0f), 127.0f);
        word |= ((uint32_t)(int)y & 0xffu) << (8 * e);
      }
      codes[c4] = word;
    }
    const int64_t crow = ((int64_t)page * 2 + plane) * page_size + off;
    unsigned char* dst = cache + (crow * hkv + kvh) * D + sub * E;
    if constexpr (E == 16)
      *reinterpret_cast<uint4*>(dst) = make_uint4(codes[0], codes[1], codes[2], codes[3]);
    else
      *reinterpret_cast<uint2*>(dst) = make_uint2(codes[0], codes[1]);
    if (sub == 0) scales[crow * hkv + kvh] = (uint16_t)f32_to_bf16_bits(s);
  }
}

}  // namespace

// ---- FP8 KV cache (E4M3 with one static power-of-two scale: the stored value is e4m3(bf16(x * kv_scale)), the
// attended value stored / kv_scale, exact in bf16). q35_group.py:44-54, 244-247 (KV8=2).
namespace {
int check_kv_scale(float s) {
  int e = 0;
  const float m = frexpf(s, &e);
  return s > 0.f && m == 0.5f && e >= -125 && e <= 126 ? AXK_OK : AXK_E_SHAPE;  // a power of two
}
}  // namespace

extern "C" int axk_paged_decode_fp8(const uint16_t* q, const uint8_t* kv_cache, const int32_t* indptr,
                                    const int32_t* indices, const int32_t* last_page_len, uint16_t* out,
                                    int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                    int64_t page_size, int64_t num_pages, float sm_scale, float kv_scale,
                                    void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(q && kv_cache && indptr && indices && last_page_len && out, AXK_E_NULL);
  int rc = check_heads(batch, num_qo_heads, num_kv_heads, head_dim);
  if (rc != AXK_OK) return rc;
  AXK_REQUIRE(head_dim == 128 || head_dim == 256, AXK_E_SHAPE);  // whole 1 KiB load blocks split over the waves
  AXK_REQUIRE(check_kv_scale(kv_scale) == AXK_OK, AXK_E_SHAPE);
  AXK_REQUIRE(page_size >= kTile && page_size % kTile == 0 && page_size <= 4096 && num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(q, 16) && axk_aligned(kv_cache, 16), AXK_E_ALIGN);
  const size_t need = axk_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const size_t qbytes = (size_t)batch * num_qo_heads * head_dim * 2;
  AXK_REQUIRE(!axk_overlap(out, qbytes, q, qbytes), AXK_E_ALIAS);
  AXK_REQUIRE(!axk_overlap(out, qbytes, workspace, workspace_bytes), AXK_E_ALIAS);
  hipStream_t st = axk_stream(stream);
  rc = decode_plan(indptr, last_page_len, batch, num_qo_heads, num_kv_heads, head_dim, page_size, 1, 0, workspace,
                   workspace_bytes, st);
  if (rc != AXK_OK) return rc;
  const int B = (int)batch, HQ = (int)num_qo_heads, HKV = (int)num_kv_heads, PS = (int)page_size;
  rc = head_dim == 128 ? launch_split<128, 1>(q, kv_cache, indptr, last_page_len, indices, out, B, HQ, HKV, PS,
                                              num_pages, sm_scale, workspace, st, 1.0f / kv_scale)
                       : launch_split<256, 1>(q, kv_cache, indptr, last_page_len, indices, out, B, HQ, HKV, PS,
                                              num_pages, sm_scale, workspace, st, 1.0f / kv_scale);
  if (rc != AXK_OK) return rc;
  return decode_merge(indptr, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim, page_size, 1, 0,
                      workspace, st);
}

extern "C" int axk_paged_kv_write_fp8(const uint16_t* k, const uint16_t* v, uint8_t* kv_cache,
                                      const int32_t* cache_location, int64_t batch, int64_t num_kv_heads,
                                      int64_t head_dim, int64_t page_size, int64_t num_pages, float kv_scale,
                                      int32_t* status, axk_stream_t stream) {
  AXK_REQUIRE(k && v && kv_cache && cache_location, AXK_E_NULL);
  AXK_REQUIRE(batch >= 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 8 == 0, AXK_E_SHAPE);
  AXK_REQUIRE(page_size > 0 && num_pages > 0 && check_kv_scale(kv_scale) == AXK_OK, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(k, 16) && axk_aligned(v, 16) && axk_aligned(kv_cache, 8), AXK_E_ALIGN);
  if (batch == 0) return AXK_OK;
  const int64_t chunks = 2 * batch * num_kv_heads * head_dim / 8;
  int64_t grid = (chunks + 255) / 256;
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(paged_kv_write_fp8_kernel, dim3((unsigned)grid), dim3(256), 0, axk_stream(stream), k, v, kv_cache,
                     cache_location, (int)batch, (int)num_kv_heads, (int)head_dim, (int)page_size, num_pages, kv_scale,
                     status);
  return axk_launch_status();
}

// ---- INT8 KV cache with a bf16 scale per row and KV head (q35_group.py:44-47, 197-221, 250-255, KV8=1) ----
extern "C" int axk_paged_decode_i8(const uint16_t* q, const int8_t* kv_cache, const uint16_t* kv_scales,
                                   const int32_t* indptr, const int32_t* indices, const int32_t* last_page_len,
                                   uint16_t* out, int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                   int64_t head_dim, int64_t page_size, int64_t num_pages, float sm_scale,
                                   void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(q && kv_cache && kv_scales && indptr && indices && last_page_len && out, AXK_E_NULL);
  int rc = check_heads(batch, num_qo_heads, num_kv_heads, head_dim);
  if (rc != AXK_OK) return rc;
  AXK_REQUIRE(head_dim == 128 || head_dim == 256, AXK_E_SHAPE);  // whole 1 KiB load blocks split over the waves
  AXK_REQUIRE(num_kv_heads <= 16, AXK_E_SHAPE);  // the range the INT8 tests cover (HKV 1 .. 16)
  AXK_REQUIRE(page_size >= kTile && page_size % kTile == 0 && page_size <= 4096 && num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(q, 16) && axk_aligned(kv_cache, 16) && axk_aligned(kv_scales, 4), AXK_E_ALIGN);
  const size_t need = axk_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const size_t qbytes = (size_t)batch * num_qo_heads * head_dim * 2;
  AXK_REQUIRE(!axk_overlap(out, qbytes, q, qbytes), AXK_E_ALIAS);
  AXK_REQUIRE(!axk_overlap(out, qbytes, workspace, workspace_bytes), AXK_E_ALIAS);
  hipStream_t st = axk_stream(stream);
  rc = decode_plan(indptr, last_page_len, batch, num_qo_heads, num_kv_heads, head_dim, page_size, 1, 0, workspace,
                   workspace_bytes, st);
  if (rc != AXK_OK) return rc;
  const int B = (int)batch, HQ = (int)num_qo_heads, HKV = (int)num_kv_heads, PS = (int)page_size;
  rc = head_dim == 128 ? launch_split<128, 1, 1>(q, kv_cache, indptr, last_page_len, indices, out, B, HQ, HKV, PS,
                                                 num_pages, sm_scale, workspace, st, 1.0f, 0, kv_scales)
                       : launch_split<256, 1, 1>(q, kv_cache, indptr, last_page_len, indices, out, B, HQ, HKV, PS,
                                                 num_pages, sm_scale, workspace, st, 1.0f, 0, kv_scales);
  if (rc != AXK_OK) return rc;
  return decode_merge(indptr, last_page_len, out, batch, num_qo_heads, num_kv_heads, head_dim, page_size, 1, 0,
                      workspace, st);
}

extern "C" int axk_paged_kv_write_i8(const uint16_t* k, const uint16_t* v, int8_t* kv_cache, uint16_t* kv_scales,
                                     const int32_t* cache_location, int64_t batch, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t page_size, int64_t num_pages, int32_t* status,
                                     axk_stream_t stream) {
  AXK_REQUIRE(k && v && kv_cache && kv_scales && cache_location, AXK_E_NULL);
  AXK_REQUIRE(batch >= 0 && num_kv_heads > 0 && (head_dim == 128 || head_dim == 256), AXK_E_SHAPE);
  AXK_REQUIRE(page_size > 0 && num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(k, 16) && axk_aligned(v, 16) && axk_aligned(kv_cache, 16) && axk_aligned(kv_scales, 2),
              AXK_E_ALIGN);
  if (batch == 0) return AXK_OK;
  const int64_t threads = 2 * batch * num_kv_heads * 16;
  int64_t grid = (threads + 255) / 256;
  if (grid > 4096) grid = 4096;
  auto* c8 = reinterpret_cast<unsigned char*>(kv_cache);
  if (head_dim == 128)
    hipLaunchKernelGGL(paged_kv_write_i8_kernel<128>, dim3((unsigned)grid), dim3(256), 0, axk_stream(stream), k, v,
                       c8, kv_scales, cache_location, (int)batch, (int)num_kv_heads, (int)page_size, num_pages,
                       status);
  else
    hipLaunchKernelGGL(paged_kv_write_i8_kernel<256>, dim3((unsigned)grid), dim3(256), 0, axk_stream(stream), k, v,
                       c8, kv_scales, cache_location, (int)batch, (int)num_kv_heads, (int)page_size, num_pages,
                       status);
  return axk_launch_status();
}

// Prefill / speculative-verify attention: the qo_indptr[b + 1] - qo_indptr[b] new tokens of each sequence (rows of q,
// already written into the cache as the sequence's last tokens) attend causally over its paged history and
// themselves. flash_attn.py:471-611 (paged_flash_attention: history pages, then the causal current block),
// q35_prefill.py:264-336 (the G x P-row block attention per KV head).
namespace {
// axk_paged_prefill, with the optional attention output gate applied as each row is written (gate rows ldg apart).
int prefill_impl(const uint16_t* q, const uint16_t* kv_cache, const int32_t* qo_indptr, const int32_t* indptr,
                 const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch, int64_t total_q,
                 int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pages,
                 float sm_scale, int32_t* status, hipStream_t st, const uint16_t* gate, int64_t ldg) {
  AXK_REQUIRE(q && kv_cache && qo_indptr && indptr && indices && last_page_len && out, AXK_E_NULL);
  AXK_REQUIRE(batch > 0 && batch <= (1 << 20) && total_q >= 0 && total_q <= (1 << 24), AXK_E_SHAPE);
  AXK_REQUIRE(num_kv_heads > 0 && num_qo_heads > 0 && num_qo_heads % num_kv_heads == 0, AXK_E_SHAPE);
  AXK_REQUIRE(num_kv_heads <= 4096 && total_q * num_qo_heads <= ((int64_t)1 << 31) / 256, AXK_E_SHAPE);
  AXK_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, AXK_E_SHAPE);
  AXK_REQUIRE(page_size >= kTile && page_size % kTile == 0 && page_size <= 4096 && num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(q, 16) && axk_aligned(kv_cache, 16) && axk_aligned(out, 8), AXK_E_ALIGN);
  if (total_q == 0) return AXK_OK;
  const size_t qbytes = (size_t)total_q * num_qo_heads * head_dim * 2;
  AXK_REQUIRE(!axk_overlap(out, qbytes, q, qbytes), AXK_E_ALIAS);
  const int B = (int)batch, T = (int)total_q, HQ = (int)num_qo_heads, HKV = (int)num_kv_heads, PS = (int)page_size;
  switch (head_dim) {
    case 64:
      return launch_prefill<64>(q, kv_cache, qo_indptr, indptr, last_page_len, indices, out, B, T, HQ, HKV, PS,
                                num_pages, sm_scale, status, st, gate, ldg);
    case 128:
      return launch_prefill<128>(q, kv_cache, qo_indptr, indptr, last_page_len, indices, out, B, T, HQ, HKV, PS,
                                 num_pages, sm_scale, status, st, gate, ldg);
    default:
      return launch_prefill<256>(q, kv_cache, qo_indptr, indptr, last_page_len, indices, out, B, T, HQ, HKV, PS,
                                 num_pages, sm_scale, status, st, gate, ldg);
  }
}
}  // namespace

extern "C" int axk_paged_prefill(const uint16_t* q, const uint16_t* kv_cache, const int32_t* qo_indptr,
                                 const int32_t* indptr, const int32_t* indices, const int32_t* last_page_len,
                                 uint16_t* out, int64_t batch, int64_t total_q, int64_t num_qo_heads,
                                 int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pages,
                                 float sm_scale, int32_t* status, axk_stream_t stream) {
  return prefill_impl(q, kv_cache, qo_indptr, indptr, indices, last_page_len, out, batch, total_q, num_qo_heads,
                      num_kv_heads, head_dim, page_size, num_pages, sm_scale, status, axk_stream(stream), nullptr, 0);
}

int axk_paged_prefill_gated(const uint16_t* q, const uint16_t* kv_cache, const int32_t* qo_indptr,
                            const int32_t* indptr, const int32_t* indices, const int32_t* last_page_len,
                            const uint16_t* gate, int64_t ldg, uint16_t* out, int64_t batch, int64_t total_q,
                            int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                            int64_t num_pages, float sm_scale, hipStream_t stream) {
  AXK_REQUIRE(gate, AXK_E_NULL);
  AXK_REQUIRE(ldg >= head_dim, AXK_E_SHAPE);
  if (total_q > 0) {
    const size_t gbytes = (size_t)((total_q * num_qo_heads - 1) * ldg + head_dim) * 2;
    AXK_REQUIRE(!axk_overlap(out, (size_t)total_q * num_qo_heads * head_dim * 2, gate, gbytes), AXK_E_ALIAS);
  }
  return prefill_impl(q, kv_cache, qo_indptr, indptr, indices, last_page_len, out, batch, total_q, num_qo_heads,
                      num_kv_heads, head_dim, page_size, num_pages, sm_scale, nullptr, stream, gate, ldg);
}
