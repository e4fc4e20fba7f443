// Paged flash-attention decode (split-KV, GQA) and the paged KV write, for gfx950.
//
// KV cache layout (sgl_kernel_axera/attention/flash_attn.py:55): cache[P, 2, page_size, HKV, D] bf16,
// plane 0 = K, plane 1 = V. Page table in CSR form: the pages of sequence b are
// indices[indptr[b] .. indptr[b+1]); the last one holds last_page_len[b] valid tokens (1..page_size),
// every other page is full (flash_attn.py:1421-1596 page-id lookup, tail mask 87-104).
//
// Two kernels:
//  1. plan   — one wave: pages per split so that the number of (sequence, KV head, split) work items
//              is about kTargetItems; prefix offsets of the items per sequence; zeroes the arrival
//              counters. Depends only on the page-table shape, so one plan serves every attention layer
//              of a decode step (no host sync, no memset: graph-capturable).
//  2. decode — one workgroup per work item. Each wave takes 32-token tiles of the item's pages:
//              S^T = K Q^T on MFMA (K rows straight from HBM with 128-bit loads, Q in registers),
//              online softmax in fp32 (exp2 domain), P (bf16) x V on MFMA with V staged through a
//              padded LDS tile (the token-contiguous operand MFMA needs); the 4 waves merge their
//              (m, l, O) in LDS. A sequence with one split writes its output directly; otherwise the
//              item writes an fp32 partial and the last item of its (sequence, KV head) to arrive
//              (atomic counter) merges all partials by log-sum-exp — the split-KV merge of
//              models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:330-349 — and resets the counter.
#include "axk_common.h"
#include "axk_host.h"

namespace {

constexpr int kWaves = 4;
constexpr int kTile = 32;  // tokens per tile = one PV MFMA k-step
constexpr int kTargetItems = 1024;
constexpr int kMaxGroup = 16;  // query heads per KV head (MFMA N tile)
constexpr float kLog2e = 1.4426950408889634f;

struct PlanHeader {
  int n_items;
  int pages_per_split;
  int bad_page;  // set to 1 if a page id outside [0, num_pages) was met (page skipped)
  int batch;     // batch / num_kv_heads the plan was made for (checked by the run kernel)
  int hkv;
  int pad[3];
};

size_t ws_items_max(int64_t batch, int64_t hkv) { return (size_t)kTargetItems + (size_t)batch * hkv; }

size_t ws_layout(int64_t batch, int64_t hkv, int64_t group, int64_t d, size_t* off_item, size_t* off_cnt,
                 size_t* off_m, size_t* off_l, size_t* off_o) {
  const size_t maxi = ws_items_max(batch, hkv);
  size_t off = sizeof(PlanHeader);
  *off_item = off;
  off += sizeof(int) * (size_t)(batch + 1);
  *off_cnt = off;
  off += sizeof(int) * (size_t)(batch * hkv);
  off = (off + 255) & ~(size_t)255;
  *off_m = off;
  off += sizeof(float) * maxi * group;
  *off_l = off;
  off += sizeof(float) * maxi * group;
  off = (off + 255) & ~(size_t)255;
  *off_o = off;
  off += sizeof(float) * maxi * group * d;
  return off;
}

__global__ __launch_bounds__(64) void paged_plan_kernel(const int* __restrict__ indptr, int batch, int hkv,
                                                        PlanHeader* __restrict__ hdr, int* __restrict__ item_off,
                                                        int* __restrict__ counters) {
  const int lane = threadIdx.x;
  for (int i = lane; i < batch * hkv; i += 64) counters[i] = 0;
  // total pages
  int tot = 0;
  for (int b = lane; b < batch; b += 64) tot += indptr[b + 1] - indptr[b];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
  const long long work = (long long)tot * hkv;
  int pps = (int)((work + kTargetItems - 1) / kTargetItems);
  if (pps < 1) pps = 1;
  // prefix sum of items per sequence, 64 sequences at a time
  int base = 0;
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const int b = b0 + lane;
    int cnt = 0;
    if (b < batch) {
      const int np = indptr[b + 1] - indptr[b];
      cnt = hkv * ((np + pps - 1) / pps);
    }
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    if (b < batch) item_off[b] = base + incl - cnt;
    base += __shfl(incl, 63, 64);
  }
  if (lane == 0) {
    item_off[batch] = base;
    hdr->n_items = base;
    hdr->pages_per_split = pps;
    hdr->bad_page = 0;
    hdr->batch = batch;
    hdr->hkv = hkv;
  }
}

template <int D>
struct PagedCfg {
  static constexpr int KSTEPS = D / 32;         // MFMA k-steps over the head dim
  static constexpr int DQ = D / 4;              // head-dim values per lane group
  static constexpr int DT = D / 16;             // 16-wide d tiles of O
  static constexpr int ROW = D * 2 + 16;        // LDS bytes per staged V row: 16-byte aligned rows, and
                                                // the 4 lane groups reading rows 4g + i hit disjoint banks
  static constexpr int VBYTES = kTile * ROW;    // one wave's V tile
  static constexpr int CHUNKS = D / 8;          // 16-byte chunks per row
};

template <int D>
__global__ __launch_bounds__(256) void paged_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ cache, const int* __restrict__ indptr,
    const int* __restrict__ indices, const int* __restrict__ last_page_len, int batch, int hq, int hkv,
    int page_size, int64_t num_pages, float sm_scale, PlanHeader* __restrict__ hdr,
    const int* __restrict__ item_off, int* __restrict__ counters, float* __restrict__ part_m,
    float* __restrict__ part_l, float* __restrict__ part_o, uint16_t* __restrict__ out) {
  using C = PagedCfg<D>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int it = blockIdx.x;
  const int n_items = hdr->n_items;
  if (it >= n_items || hdr->batch != batch || hdr->hkv != hkv) return;
  const int pps = hdr->pages_per_split;
  const int group = hq / hkv;

  // item -> (b, kvh, split): binary search over the per-sequence item offsets
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (item_off[mid] <= it) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int nsplit = (item_off[b + 1] - item_off[b]) / hkv;
  const int local = it - item_off[b];
  const int kvh = local / nsplit, split = local - kvh * nsplit;
  const int pbeg = indptr[b];
  const int npages = indptr[b + 1] - pbeg;
  const int lp0 = split * pps;
  const int lp1 = min(npages, lp0 + pps);
  const int last_valid = last_page_len[b];
  const int tpp = page_size / kTile;  // tiles per page
  const int ntiles = (lp1 - lp0) * tpp;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const float c = sm_scale * kLog2e;

  // Q as the B operand of S^T = K Q^T: lane (head l16, group g) holds d = g*DQ + 8s .. +8.
  axk_bf16x8 qb[C::KSTEPS];
  {
    const bool hv = l16 < group;
    const uint16_t* qp = q + ((int64_t)b * hq + kvh * group + (hv ? l16 : 0)) * D + g * C::DQ;
#pragma unroll
    for (int s = 0; s < C::KSTEPS; ++s) qb[s] = hv ? load_bf16x8(qp + 8 * s) : zero_bf16x8();
  }

  axk_f32x4 o[C::DT];
#pragma unroll
  for (int t = 0; t < C::DT; ++t) o[t] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // for head l16 (replicated over g)

  unsigned char* vt = smem + wave * C::VBYTES;
  const int64_t row_stride = (int64_t)hkv * D;          // elements between consecutive tokens
  const int64_t plane_stride = (int64_t)page_size * row_stride;

  for (int ti = wave; ti < ntiles; ti += kWaves) {
    const int lp = lp0 + ti / tpp, tp = ti - (ti / tpp) * tpp;
    const int page = indices[pbeg + lp];
    const int valid_in_page = (lp == npages - 1) ? last_valid : page_size;
    const int nvalid = min(kTile, valid_in_page - tp * kTile);
    if (nvalid <= 0) continue;
    if (page < 0 || page >= num_pages) {
      if (lane == 0) hdr->bad_page = 1;
      continue;
    }
    const uint16_t* kbase = cache + (int64_t)page * 2 * plane_stride + (int64_t)(tp * kTile) * row_stride + kvh * D;
    const uint16_t* vbase = kbase + plane_stride;

    // K rows for the two 16-token halves (A operand): lane (token l16, group g), d = g*DQ + 8s.
    axk_bf16x8 ka[2][C::KSTEPS];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int tok = 16 * h + l16;
      const bool ok = tok < nvalid;
      const uint16_t* kp = kbase + (int64_t)tok * row_stride + g * C::DQ;
#pragma unroll
      for (int s = 0; s < C::KSTEPS; ++s) ka[h][s] = ok ? load_bf16x8(kp + 8 * s) : zero_bf16x8();
    }
    // V tile -> LDS (row-major, padded); rows past nvalid are zero so masked P never meets garbage.
#pragma unroll
    for (int i = 0; i < (kTile * C::CHUNKS) / 64; ++i) {
      const int qi = i * 64 + lane;
      const int tok = qi / C::CHUNKS, ch = qi - tok * C::CHUNKS;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (tok < nvalid) v = *reinterpret_cast<const uint4*>(vbase + (int64_t)tok * row_stride + ch * 8);
      *reinterpret_cast<uint4*>(vt + tok * C::ROW + ch * 16) = v;
    }

    // S^T tiles: lane holds S[token 16h + 4g + r][head l16]
    axk_f32x4 st[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      st[h] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < C::KSTEPS; ++s) st[h] = mfma_bf16_16x16x32(ka[h][s], qb[s], st[h]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 16 * h + 4 * g + r;
        const float sv = tok < nvalid ? st[h][r] * c : -INFINITY;
        st[h][r] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);
    float psum = 0.f;
    axk_bf16x8 pa;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2f(st[h][r] - m_new);
        psum += p;
        pa[4 * h + r] = (__bf16)p;
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // O rows are heads 4g + r: fetch their alpha from lane (4g + r)
    float ar[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r, 64);

    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // P x V: B operand lane (d = 16t + l16, group g) = V[token(8g + i)][d], token(8g+i) matching pa's order
#pragma unroll
    for (int t = 0; t < C::DT; ++t) {
      axk_bf16x8 vb;
      const unsigned char* col = vt + (16 * t + l16) * 2;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int tok = (i < 4) ? (4 * g + i) : (16 + 4 * g + i - 4);
        vb[i] = *reinterpret_cast<const __bf16*>(col + tok * C::ROW);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) o[t][r] *= ar[r];
      o[t] = mfma_bf16_16x16x32(pa, vb, o[t]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the 4 waves' (m, l, O) in LDS, write the item partial ----
  __syncthreads();
  float* sm_m = reinterpret_cast<float*>(smem);           // [kWaves][16]
  float* sm_l = sm_m + kWaves * 16;                       // [kWaves][16]
  float* sm_o = sm_l + kWaves * 16;                       // [kWaves][16][D]
  if (lane < 16) {
    sm_m[wave * 16 + lane] = m_run;
    sm_l[wave * 16 + lane] = l_run;
  }
  __syncthreads();
  // each wave rescales its O rows (heads 4g + r) to the common max
  float scale_r[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * g + r;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm_m[w * 16 + hh]);
    const float mw = sm_m[wave * 16 + hh];
    scale_r[r] = (mw == -INFINITY) ? 0.f : exp2f(mw - mm);
  }
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm_o[(wave * 16 + 4 * g + r) * D + 16 * t + l16] = o[t][r] * scale_r[r];
  __syncthreads();
  // merged (m, l) of this item for head hh
  float* sm_mm = sm_o + kWaves * 16 * D;  // [16] item max, [16] item sum
  if (threadIdx.x < 16) {
    const int hh = threadIdx.x;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm_m[w * 16 + hh]);
    float ll = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = sm_m[w * 16 + hh];
      if (mw != -INFINITY) ll += sm_l[w * 16 + hh] * exp2f(mw - mm);
    }
    sm_mm[hh] = mm;
    sm_mm[16 + hh] = ll;
  }
  __syncthreads();
  const int64_t out_base = ((int64_t)b * hq + kvh * group) * D;
  if (nsplit == 1) {  // the whole sequence in one item: normalise and store
    for (int idx = threadIdx.x; idx < group * D; idx += blockDim.x) {
      const int hh = idx / D, d = idx - hh * D;
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) acc += sm_o[(w * 16 + hh) * D + d];
      const float ll = sm_mm[16 + hh];
      out[out_base + idx] = (uint16_t)f32_to_bf16_bits(ll > 0.f ? acc / ll : 0.f);
    }
    return;
  }
  for (int idx = threadIdx.x; idx < group * D; idx += blockDim.x) {
    const int hh = idx / D, d = idx - hh * D;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) acc += sm_o[(w * 16 + hh) * D + d];
    part_o[((int64_t)it * group + hh) * D + d] = acc;
  }
  if (threadIdx.x < group) {
    part_m[(int64_t)it * group + threadIdx.x] = sm_mm[threadIdx.x];
    part_l[(int64_t)it * group + threadIdx.x] = sm_mm[16 + threadIdx.x];
  }
  // arrival: the last item of (b, kvh) merges every split of it
  __threadfence();
  __syncthreads();
  int* ticket = reinterpret_cast<int*>(sm_mm + 32);
  if (threadIdx.x == 0) *ticket = atomicAdd(&counters[b * hkv + kvh], 1);
  __syncthreads();
  if (*ticket != nsplit - 1) return;
  __threadfence();
  const int i0 = item_off[b] + kvh * nsplit;
  for (int idx = threadIdx.x; idx < group * D; idx += blockDim.x) {
    const int hh = idx / D, d = idx - hh * D;
    float mm = -INFINITY;
    for (int i = 0; i < nsplit; ++i) mm = fmaxf(mm, __builtin_nontemporal_load(&part_m[(int64_t)(i0 + i) * group + hh]));
    float ll = 0.f, acc = 0.f;
    for (int i = 0; i < nsplit; ++i) {
      const float mi = __builtin_nontemporal_load(&part_m[(int64_t)(i0 + i) * group + hh]);
      if (mi == -INFINITY) continue;
      const float w = exp2f(mi - mm);
      ll += __builtin_nontemporal_load(&part_l[(int64_t)(i0 + i) * group + hh]) * w;
      acc += __builtin_nontemporal_load(&part_o[((int64_t)(i0 + i) * group + hh) * D + d]) * w;
    }
    out[out_base + idx] = (uint16_t)f32_to_bf16_bits(ll > 0.f ? acc / ll : 0.f);
  }
  if (threadIdx.x == 0) counters[b * hkv + kvh] = 0;  // ready for another run with the same plan
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

struct WsView {
  PlanHeader* hdr;
  int* item_off;
  int* counters;
  float *pm, *pl, *po;
};

WsView ws_view(void* ws, int batch, int hkv, int group, int d) {
  size_t oi, oc, om, ol, oo;
  ws_layout(batch, hkv, group, d, &oi, &oc, &om, &ol, &oo);
  unsigned char* w = reinterpret_cast<unsigned char*>(ws);
  return {reinterpret_cast<PlanHeader*>(w), reinterpret_cast<int*>(w + oi), reinterpret_cast<int*>(w + oc),
          reinterpret_cast<float*>(w + om), reinterpret_cast<float*>(w + ol), reinterpret_cast<float*>(w + oo)};
}

template <int D>
int launch_run(const uint16_t* q, const uint16_t* cache, const int* indptr, const int* indices,
               const int* last_page_len, uint16_t* out, int batch, int hq, int hkv, int page_size, int64_t num_pages,
               float sm_scale, void* ws, hipStream_t st) {
  const int group = hq / hkv;
  const WsView v = ws_view(ws, batch, hkv, group, D);
  const size_t lds_v = (size_t)kWaves * PagedCfg<D>::VBYTES;
  const size_t lds_m = sizeof(float) * (2 * kWaves * 16 + (size_t)kWaves * 16 * D + 32 + 4);
  const size_t lds = lds_v > lds_m ? lds_v : lds_m;
  static bool lds_raised = false;  // > 64 KiB of dynamic LDS must be allowed once per kernel
  if (!lds_raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_decode_kernel<D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return AXK_E_LAUNCH;
    lds_raised = true;
  }
  const unsigned items = (unsigned)ws_items_max(batch, hkv);
  hipLaunchKernelGGL((paged_decode_kernel<D>), dim3(items), dim3(64 * kWaves), lds, st, q, cache, indptr, indices,
                     last_page_len, batch, hq, hkv, page_size, num_pages, sm_scale, v.hdr, v.item_off, v.counters,
                     v.pm, v.pl, v.po, out);
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

extern "C" int axk_paged_decode_plan(const int32_t* indptr, int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                     int64_t head_dim, void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(indptr, AXK_E_NULL);
  const int rc = check_heads(batch, num_qo_heads, num_kv_heads, head_dim);
  if (rc != AXK_OK) return rc;
  const size_t need = axk_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const WsView v = ws_view(workspace, (int)batch, (int)num_kv_heads, (int)(num_qo_heads / num_kv_heads),
                           (int)head_dim);
  hipLaunchKernelGGL(paged_plan_kernel, dim3(1), dim3(64), 0, axk_stream(stream), indptr, (int)batch,
                     (int)num_kv_heads, v.hdr, v.item_off, v.counters);
  return axk_launch_status();
}

extern "C" int axk_paged_decode_run(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                                    const int32_t* indices, const int32_t* last_page_len, uint16_t* out,
                                    int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                    int64_t page_size, int64_t num_pages, float sm_scale, void* workspace,
                                    size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(q && kv_cache && indptr && indices && last_page_len && out, AXK_E_NULL);
  const int rc = check_heads(batch, num_qo_heads, num_kv_heads, head_dim);
  if (rc != AXK_OK) return rc;
  AXK_REQUIRE(page_size >= kTile && page_size % kTile == 0 && page_size <= 4096, AXK_E_SHAPE);
  AXK_REQUIRE(num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(q, 16) && axk_aligned(kv_cache, 16), AXK_E_ALIGN);
  const size_t need = axk_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const size_t qbytes = (size_t)batch * num_qo_heads * head_dim * 2;
  AXK_REQUIRE(!axk_overlap(out, qbytes, q, qbytes), AXK_E_ALIAS);
  AXK_REQUIRE(!axk_overlap(out, qbytes, workspace, workspace_bytes), AXK_E_ALIAS);
  hipStream_t st = axk_stream(stream);
  const int B = (int)batch, HQ = (int)num_qo_heads, HKV = (int)num_kv_heads, PS = (int)page_size;
  switch (head_dim) {
    case 64:
      return launch_run<64>(q, kv_cache, indptr, indices, last_page_len, out, B, HQ, HKV, PS, num_pages, sm_scale,
                            workspace, st);
    case 128:
      return launch_run<128>(q, kv_cache, indptr, indices, last_page_len, out, B, HQ, HKV, PS, num_pages, sm_scale,
                             workspace, st);
    default:
      return launch_run<256>(q, kv_cache, indptr, indices, last_page_len, out, B, HQ, HKV, PS, num_pages, sm_scale,
                             workspace, st);
  }
}

extern "C" int axk_paged_decode(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                                const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                                int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                int64_t num_pages, float sm_scale, void* workspace, size_t workspace_bytes,
                                axk_stream_t stream) {
  AXK_REQUIRE(q && kv_cache && indices && last_page_len && out, AXK_E_NULL);
  AXK_REQUIRE(page_size >= kTile && page_size % kTile == 0 && page_size <= 4096 && num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(q, 16) && axk_aligned(kv_cache, 16), AXK_E_ALIGN);
  const int rc = axk_paged_decode_plan(indptr, batch, num_qo_heads, num_kv_heads, head_dim, workspace,
                                       workspace_bytes, stream);
  if (rc != AXK_OK) return rc;
  return axk_paged_decode_run(q, kv_cache, indptr, indices, last_page_len, out, batch, num_qo_heads, num_kv_heads,
                              head_dim, page_size, num_pages, sm_scale, workspace, workspace_bytes, stream);
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
  hipLaunchKernelGGL(paged_kv_write_kernel, dim3((unsigned)grid), dim3(256), 0, axk_stream(stream), k, v, kv_cache,
                     cache_location, (int)batch, (int)num_kv_heads, (int)head_dim, (int)page_size, num_pages, status);
  return axk_launch_status();
}
