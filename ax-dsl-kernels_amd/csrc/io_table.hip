// IO tables of the roles libaxk serves: [name, bytes, dtype, shape] per input and output, as the AX engine reports a
// kernel's IO (tools/board/iojson.c:23-34) and manifest.json records it (tools/manifest/mkmanifest.py:183-199).
// Host code only.
#include <string.h>

#include <initializer_list>

#include "axk_host.h"

namespace {

// Storage bytes of n elements of an AX dtype (E2M1 packs two values per byte).
int64_t storage_bytes(int dt, int64_t n) {
  switch (dt) {
    case AXK_DT_FP4: return n / 2;
    case AXK_DT_BF16:
    case AXK_DT_F16: return 2 * n;
    case AXK_DT_F32:
    case AXK_DT_I32: return 4 * n;
    default: return n;  // u8, E4M3, E5M2, E8M0
  }
}

struct Table {
  axk_io_entry* e;
  int cap;
  int n = 0;
  bool bad = false;  // a name or rank that does not fit an entry

  void add(bool out, const char* name, int dt, std::initializer_list<int64_t> shape) {
    if (n < cap) {
      axk_io_entry& r = e[n];
      memset(&r, 0, sizeof r);
      const size_t len = strlen(name);
      if (len >= AXK_IO_NAME_MAX || shape.size() > AXK_IO_RANK_MAX) bad = true;
      memcpy(r.name, name, len < AXK_IO_NAME_MAX ? len : AXK_IO_NAME_MAX - 1);
      r.dtype = dt;
      r.output = out ? 1 : 0;
      r.rank = (int32_t)(shape.size() < AXK_IO_RANK_MAX ? shape.size() : AXK_IO_RANK_MAX);
      int64_t numel = 1;
      int i = 0;
      for (int64_t d : shape) {
        if (i < AXK_IO_RANK_MAX) r.shape[i++] = d;
        numel *= d;
      }
      r.bytes = storage_bytes(dt, numel);
    }
    ++n;
  }
  void in(const char* name, int dt, std::initializer_list<int64_t> shape) { add(false, name, dt, shape); }
  void out(const char* name, int dt, std::initializer_list<int64_t> shape) { add(true, name, dt, shape); }

  // The weight w_<x> [rows, k] and its scales s_<x> in weight format fmt (AXK_WFMT_*).
  void weight(const char* x, int64_t rows, int64_t k, int fmt) {
    char w[AXK_IO_NAME_MAX], s[AXK_IO_NAME_MAX];
    if (strlen(x) + 3 > AXK_IO_NAME_MAX) bad = true;
    w[0] = 'w', s[0] = 's', w[1] = s[1] = '_';
    strncpy(w + 2, x, AXK_IO_NAME_MAX - 3);
    strncpy(s + 2, x, AXK_IO_NAME_MAX - 3);
    w[AXK_IO_NAME_MAX - 1] = s[AXK_IO_NAME_MAX - 1] = 0;
    if (fmt == AXK_WFMT_FP8_CHANNEL) {
      in(w, AXK_DT_FP8E4M3, {rows, k});
      in(s, AXK_DT_F32, {rows});
    } else {
      in(w, fmt == AXK_WFMT_MXFP4 ? AXK_DT_FP4 : AXK_DT_FP8E4M3, {rows, k});
      in(s, AXK_DT_U8, {rows, k / 32});
    }
  }
};

// dims[i], or def when the caller passed fewer.
struct Dims {
  const int64_t* d;
  int n;
  int64_t operator()(int i, int64_t def) const { return i < n ? d[i] : def; }
};

bool mx_fmt_ok(int64_t f) { return f == AXK_WFMT_FP8_CHANNEL || f == AXK_WFMT_MXFP8 || f == AXK_WFMT_MXFP4; }

// The dense MLP (the MoE layer's shared expert) and, with experts, the MoE layer's router and shared-expert gate.
void mlp(Table& t, int64_t h, int64_t f, int fmt, int64_t experts) {
  t.weight("gate", f, h, fmt);
  t.weight("up", f, h, fmt);
  t.weight("down", h, f, fmt);
  if (experts > 0) {
    t.in("w_router", AXK_DT_BF16, {experts, h});
    t.in("w_shg", AXK_DT_BF16, {h});
  }
}

int lm_head(Table& t, const Dims& D) {
  const int64_t n = D(0, 0), k = D(1, 0), m = D(2, 1);
  AXK_REQUIRE(D.n >= 2 && n > 0 && k > 0 && m > 0 && k % 32 == 0, AXK_E_SHAPE);
  t.in("x", AXK_DT_BF16, {m, k});
  t.in("w", AXK_DT_FP4, {n, k});
  t.in("s", AXK_DT_U8, {n, k / 32});
  t.out("out", AXK_DT_F32, {m, n});
  return AXK_OK;
}

int gdn(Table& t, const Dims& D) {
  const int64_t h = D(0, 0), nk = D(1, 0), nv = D(2, 0), f = D(3, 0), conv = D(4, 4);
  const int64_t pf = D(5, AXK_WFMT_MXFP4), mf = D(6, AXK_WFMT_MXFP4), experts = D(7, 0), b = D(8, 1);
  AXK_REQUIRE(D.n >= 4 && h > 0 && nk > 0 && nv > 0 && f > 0 && conv >= 2 && experts >= 0 && b > 0, AXK_E_SHAPE);
  AXK_REQUIRE(h % 32 == 0 && f % 32 == 0 && nv % nk == 0, AXK_E_SHAPE);
  AXK_REQUIRE(mx_fmt_ok(pf) && mx_fmt_ok(mf), AXK_E_DTYPE);
  const int64_t kd = nk * 128, vd = nv * 128, c = 2 * kd + vd;
  t.in("x", AXK_DT_BF16, {b, 1, h});
  t.in("ln1", AXK_DT_F32, {h});
  t.weight("qkv", c, h, (int)pf);
  t.weight("z", vd, h, (int)pf);
  t.weight("b", nv, h, (int)pf);
  t.weight("a", nv, h, (int)pf);
  t.in("conv_w", AXK_DT_BF16, {c, conv});
  t.in("a_log", AXK_DT_F32, {nv});
  t.in("dt_bias", AXK_DT_F32, {nv});
  t.in("norm_w", AXK_DT_F32, {128});
  t.weight("out", h, vd, (int)pf);
  t.in("ln2", AXK_DT_F32, {h});
  mlp(t, h, f, (int)mf, experts);
  if (b == 1) {
    t.in("state_in", AXK_DT_F32, {nv, 128, 128});
  } else {
    t.in("state_in", AXK_DT_F32, {b, nv, 128, 128});
  }
  t.in("conv_in", AXK_DT_BF16, {b, conv - 1, c});
  t.out("out", AXK_DT_BF16, {b, 1, h});
  if (b == 1) {
    t.out("state_out", AXK_DT_F32, {nv, 128, 128});
  } else {
    t.out("state_out", AXK_DT_F32, {b, nv, 128, 128});
  }
  t.out("conv_out", AXK_DT_BF16, {b, conv - 1, c});
  return AXK_OK;
}

int attn(Table& t, const Dims& D) {
  const int64_t h = D(0, 0), hq = D(1, 0), hkv = D(2, 0), d = D(3, 0), f = D(4, 0);
  const int64_t pf = D(5, AXK_WFMT_MXFP4), mf = D(6, AXK_WFMT_MXFP4), experts = D(7, 0), b = D(8, 1);
  const int64_t rot = D(9, 64), page = D(10, 256), pages = D(11, 1);
  AXK_REQUIRE(D.n >= 5 && h > 0 && hq > 0 && hkv > 0 && d > 0 && f > 0 && experts >= 0 && b > 0, AXK_E_SHAPE);
  AXK_REQUIRE(h % 32 == 0 && f % 32 == 0 && (hq * d) % 32 == 0 && hq % hkv == 0, AXK_E_SHAPE);
  AXK_REQUIRE(rot >= 0 && rot % 2 == 0 && rot <= d && page > 0 && pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(mx_fmt_ok(pf) && mx_fmt_ok(mf), AXK_E_DTYPE);
  t.in("x", AXK_DT_BF16, {b, 1, h});
  t.in("ln1", AXK_DT_F32, {h});
  t.weight("q", 2 * hq * d, h, (int)pf);
  t.weight("k", hkv * d, h, (int)pf);
  t.weight("v", hkv * d, h, (int)pf);
  t.in("q_norm", AXK_DT_F32, {d});
  t.in("k_norm", AXK_DT_F32, {d});
  t.weight("o", h, hq * d, (int)pf);
  t.in("ln2", AXK_DT_F32, {h});
  mlp(t, h, f, (int)mf, experts);
  t.in("cos", AXK_DT_BF16, {b, rot / 2});
  t.in("sin", AXK_DT_BF16, {b, rot / 2});
  t.in("indptr", AXK_DT_I32, {b + 1});
  t.in("indices", AXK_DT_I32, {pages});
  t.in("last_page_len", AXK_DT_I32, {b});
  t.in("cache_location", AXK_DT_I32, {b, 2});
  t.out("out", AXK_DT_BF16, {b, 1, h});
  t.out("kv_cache", AXK_DT_BF16, {pages, 2, page, hkv, d});
  return AXK_OK;
}

int experts(Table& t, const Dims& D) {
  const int64_t e = D(0, 0), h = D(1, 0), f = D(2, 0);
  AXK_REQUIRE(D.n >= 3 && e > 0 && h > 0 && f > 0 && h % 32 == 0 && f % 32 == 0, AXK_E_SHAPE);
  t.in("e_gw", AXK_DT_U8, {e, 2 * f, h / 2});
  t.in("e_gs", AXK_DT_U8, {e, 2 * f, h / 32});
  t.in("e_dw", AXK_DT_U8, {e, h, f / 2});
  t.in("e_ds", AXK_DT_U8, {e, h, f / 32});
  return AXK_OK;
}

}  // namespace

extern "C" int axk_io_table(const char* role, const int64_t* dims, int ndims, axk_io_entry* entries, int capacity,
                            int* count) {
  AXK_REQUIRE(role && count && (ndims == 0 || dims) && ndims >= 0 && capacity >= 0, AXK_E_NULL);
  AXK_REQUIRE(capacity == 0 || entries, AXK_E_NULL);
  Table t{entries, capacity};
  const Dims D{dims, ndims};
  int st;
  if (!strcmp(role, "lm_head")) {
    st = lm_head(t, D);
  } else if (!strcmp(role, "layer.gdn")) {
    st = gdn(t, D);
  } else if (!strcmp(role, "layer.attn")) {
    st = attn(t, D);
  } else if (!strcmp(role, "experts")) {
    st = experts(t, D);
  } else {
    return AXK_E_ROLE;
  }
  if (st != AXK_OK) return st;
  *count = t.n;
  AXK_REQUIRE(!t.bad, AXK_E_SHAPE);
  return t.n > capacity ? AXK_E_BUFFER : AXK_OK;
}
