// sdq_ops_block.cpp -- C ABI of the ops around the quantized linears in a
// Flux block: MLX's fused layer/RMS norm and scaled dot-product attention
// (mlx.rs:212-238), and the fused Flux forms norm_modulate, rotate and the
// whole q/k/v -> attention -> merged heads sequence (flux.rs:165-205,
// 255-275, 300-327, 352-381, 446-461).  Validation mirrors the reference's
// callers: a status and a message, never an abort.
#include <cmath>
#include <cstring>
#include <string>

#include "kernels/launch.hpp"
#include "sdq_internal.hpp"

namespace sdq {
namespace {

std::unique_ptr<ArrayImpl> to_bf16(const ArrayImpl *a, const StreamImpl *st) {
  auto out = make_array(a->shape, SDQ_BFLOAT16, *st);
  kern::astype(a->data(), a->dtype, out->data(), SDQ_BFLOAT16, int64_t(a->size), st->stream);
  return out;
}

// A norm parameter: absent, or C values of a float dtype.
const ArrayImpl *norm_param(sdq_array p, const char *op, const char *name, int C, const StreamImpl *st) {
  if (!p.ctx) return nullptr;
  ArrayImpl *a = array_of(p, op, name);
  same_device(a, st, name);
  if (!is_float_dtype(a->dtype)) fail(std::string("`") + name + "` must be a float array");
  if (int64_t(a->size) != C)
    fail(std::string("`") + name + "` has " + std::to_string(a->size) + " values, the last axis has " +
         std::to_string(C));
  order_after(a, st);
  return a;
}

int param_dtype(const ArrayImpl *a, const ArrayImpl *b) {
  if (a && b && a->dtype != b->dtype) fail("weight and bias must have one dtype");
  return a ? a->dtype : b ? b->dtype : SDQ_FLOAT32;
}

ArrayImpl *float_input(sdq_array x, const char *op, const char *name, const StreamImpl *st) {
  ArrayImpl *a = array_of(x, op, name);
  same_device(a, st, name);
  if (!is_float_dtype(a->dtype))
    fail(std::string("`") + name + "` must be float32, bfloat16 or float16, got " + dtype_name(a->dtype));
  order_after(a, st);
  return a;
}

} // namespace
} // namespace sdq

using namespace sdq;

extern "C" {

int sdq_fast_layer_norm(sdq_array *res, sdq_array x, sdq_array weight, sdq_array bias, float eps, sdq_stream s) {
  SDQ_GUARD("layer_norm", {
    StreamImpl *st = stream_of(s, "layer_norm");
    if (!res) fail("result pointer is NULL");
    ArrayImpl *xa = float_input(x, "layer_norm", "x", st);
    if (xa->shape.empty()) fail("layer_norm needs at least one axis");
    const int C = xa->shape.back();
    const ArrayImpl *w = norm_param(weight, "layer_norm", "weight", C, st);
    const ArrayImpl *b = norm_param(bias, "layer_norm", "bias", C, st);
    auto out = make_array(xa->shape, xa->dtype, *st);
    const int64_t rows = C ? int64_t(xa->size) / C : 0;
    kern::layer_norm(xa->data(), xa->dtype, out->data(), xa->dtype, rows, C, eps, w ? w->data() : nullptr,
                     b ? b->data() : nullptr, param_dtype(w, b), st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_fast_rms_norm(sdq_array *res, sdq_array x, sdq_array weight, float eps, sdq_stream s) {
  SDQ_GUARD("rms_norm", {
    StreamImpl *st = stream_of(s, "rms_norm");
    if (!res) fail("result pointer is NULL");
    ArrayImpl *xa = float_input(x, "rms_norm", "x", st);
    if (xa->shape.empty()) fail("rms_norm needs at least one axis");
    const int C = xa->shape.back();
    const ArrayImpl *w = norm_param(weight, "rms_norm", "weight", C, st);
    auto out = make_array(xa->shape, xa->dtype, *st);
    const int64_t rows = C ? int64_t(xa->size) / C : 0;
    kern::rms_norm(xa->data(), xa->dtype, out->data(), xa->dtype, rows, C, eps, w ? w->data() : nullptr,
                   param_dtype(w, nullptr), st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_flux_norm_modulate(sdq_array *res, sdq_array x, sdq_array shift, sdq_array scale, float eps,
                           sdq_stream s) {
  SDQ_GUARD("norm_modulate", {
    StreamImpl *st = stream_of(s, "norm_modulate");
    if (!res) fail("result pointer is NULL");
    ArrayImpl *xa = float_input(x, "norm_modulate", "x", st);
    if (xa->shape.size() != 3) fail("norm_modulate takes x as [batch, tokens, channels], got " + shape_str(xa->shape));
    const int B = xa->shape[0], N = xa->shape[1], C = xa->shape[2];
    ArrayImpl *sh = float_input(shift, "norm_modulate", "shift", st);
    ArrayImpl *sc = float_input(scale, "norm_modulate", "scale", st);
    for (const ArrayImpl *p : {sh, sc})
      if (int64_t(p->size) != int64_t(B) * C)
        fail("norm_modulate: shift and scale must hold [batch, 1, channels] = " + std::to_string(B) + " x " +
             std::to_string(C) + " values, got " + shape_str(p->shape));
    if (sh->dtype != sc->dtype) fail("norm_modulate: shift and scale must have one dtype");
    auto out = make_array(xa->shape, xa->dtype, *st);
    kern::norm_modulate(xa->data(), xa->dtype, out->data(), xa->dtype, int64_t(B) * N, C, eps, sh->data(),
                        sc->data(), sh->dtype, N ? N : 1, st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_flux_rope(sdq_array *res, sdq_array x, sdq_array cos, sdq_array sin, sdq_stream s) {
  SDQ_GUARD("rope", {
    StreamImpl *st = stream_of(s, "rope");
    if (!res) fail("result pointer is NULL");
    ArrayImpl *xa = float_input(x, "rope", "x", st);
    if (xa->shape.size() != 4) fail("mlx: rope got " + shape_str(xa->shape));
    const int N = xa->shape[2], D = xa->shape[3];
    if (D % 2 != 0) fail("rope: head_dim must be even, got " + std::to_string(D));
    ArrayImpl *ca = float_input(cos, "rope", "cos", st);
    ArrayImpl *sa = float_input(sin, "rope", "sin", st);
    for (const ArrayImpl *p : {ca, sa}) {
      if (p->dtype != SDQ_FLOAT32) fail("rope: cos and sin must be float32 tables");
      if (int64_t(p->size) != int64_t(N) * (D / 2))
        fail("rope: cos and sin must hold [1, " + std::to_string(N) + ", " + std::to_string(D / 2) +
             "] values, got " + shape_str(p->shape));
    }
    auto out = make_array(xa->shape, xa->dtype, *st);
    kern::rope(xa->data(), xa->dtype, out->data(), int64_t(xa->size) / D, D, N,
               static_cast<const float *>(ca->data()), static_cast<const float *>(sa->data()), st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_fast_scaled_dot_product_attention(sdq_array *res, sdq_array queries, sdq_array keys, sdq_array values,
                                          float scale, const char *mask_mode, sdq_array mask_arr,
                                          sdq_array sinks, sdq_stream s) {
  SDQ_GUARD("scaled_dot_product_attention", {
    StreamImpl *st = stream_of(s, "scaled_dot_product_attention");
    if (!res) fail("result pointer is NULL");
    const char *op = "scaled_dot_product_attention";
    ArrayImpl *q = float_input(queries, op, "queries", st);
    ArrayImpl *k = float_input(keys, op, "keys", st);
    ArrayImpl *v = float_input(values, op, "values", st);
    if (sinks.ctx) fail("attention sinks are not supported");
    for (const ArrayImpl *a : {q, k, v})
      if (a->shape.size() != 4)
        fail("queries, keys and values must be [batch, heads, seq, head_dim], got " + shape_str(a->shape));
    const int B = q->shape[0], Hq = q->shape[1], Nq = q->shape[2], D = q->shape[3];
    const int Hk = k->shape[1], Nk = k->shape[2];
    if (k->shape[0] != B || v->shape[0] != B || v->shape[1] != Hk || v->shape[2] != Nk || k->shape[3] != D)
      fail("keys and values must match the queries: q " + shape_str(q->shape) + ", k " + shape_str(k->shape) +
           ", v " + shape_str(v->shape));
    if (v->shape[3] != D) fail("values must have the queries' head_dim");
    if (D != 64 && D != 128) fail("head_dim " + std::to_string(D) + " is not supported (64 or 128)");
    if (Hk == 0 || Hq % Hk != 0) fail("the query heads must be a multiple of the key/value heads");
    if (Nk == 0) fail("attention over zero keys");

    kern::AttnArgs a;
    const std::string mode = mask_mode ? mask_mode : "";
    const ArrayImpl *mask = nullptr;
    if (mode.empty()) {
      a.mode = 0;
    } else if (mode == "causal") {
      a.mode = 1;
      a.causal_offset = Nk - Nq;
    } else if (mode == "array") {
      a.mode = 2;
      if (!mask_arr.ctx) fail("mask_mode 'array' needs a mask");
      mask = float_input(mask_arr, op, "mask", st);
      const auto &ms = mask->shape;
      if (ms.empty() || ms.size() > 4) fail("the mask must have 1 to 4 axes, got " + shape_str(ms));
      if (ms.back() != Nk) fail("the mask's last axis must be the key length " + std::to_string(Nk));
      // Right-align against [B, Hq, Nq, Nk]; size-1 axes broadcast.
      const int full[4] = {B, Hq, Nq, Nk};
      int dims[4] = {1, 1, 1, 1};
      for (size_t i = 0; i < ms.size(); ++i) dims[4 - ms.size() + i] = ms[i];
      for (int i = 0; i < 3; ++i)
        if (dims[i] != 1 && dims[i] != full[i])
          fail("the mask " + shape_str(ms) + " does not broadcast to the scores [" + std::to_string(B) + ", " +
               std::to_string(Hq) + ", " + std::to_string(Nq) + ", " + std::to_string(Nk) + "]");
      a.m_sq = dims[2] == 1 ? 0 : Nk;
      a.m_sh = dims[1] == 1 ? 0 : int64_t(dims[2]) * Nk;
      a.m_sb = dims[0] == 1 ? 0 : int64_t(dims[1]) * dims[2] * Nk;
      a.mask = mask->data();
      a.mask_dtype = mask->dtype;
    } else {
      fail("mask_mode must be '', 'causal' or 'array', got '" + mode + "'");
    }

    std::unique_ptr<ArrayImpl> qb, kb;
    const ArrayImpl *qx = q, *kx = k;
    if (q->dtype != SDQ_BFLOAT16) qx = (qb = to_bf16(q, st)).get();
    if (k->dtype != SDQ_BFLOAT16) kx = (kb = to_bf16(k, st)).get();
    const int64_t ldt = kern::attention_vt_stride(Nk);
    auto vt = make_array({B * Hk, D, int(ldt)}, SDQ_BFLOAT16, *st);
    kern::transpose_v(v->data(), v->dtype, int64_t(B) * Hk, Nk, D, int64_t(Nk) * D, D,
                      static_cast<uint16_t *>(vt->data()), int64_t(D) * ldt, ldt, st->stream);
    auto out = make_array(q->shape, q->dtype, *st);
    a.q = static_cast<const uint16_t *>(qx->data());
    a.k = static_cast<const uint16_t *>(kx->data());
    a.vt = static_cast<const uint16_t *>(vt->data());
    a.o = out->data();
    a.q_sn = D, a.q_sh = int64_t(Nq) * D, a.q_sb = int64_t(Hq) * Nq * D;
    a.k_sn = D, a.k_sh = int64_t(Nk) * D, a.k_sb = int64_t(Hk) * Nk * D;
    a.v_sd = ldt, a.v_sh = int64_t(D) * ldt, a.v_sb = int64_t(Hk) * D * ldt;
    a.o_sn = D, a.o_sh = int64_t(Nq) * D, a.o_sb = int64_t(Hq) * Nq * D;
    a.B = B, a.H = Hq, a.group = Hq / Hk, a.Nq = Nq, a.Nk = Nk, a.D = D;
    a.scale_log2 = scale * 1.4426950408889634f;
    kern::attention(a, q->dtype, st->stream);
    set_result(res, std::move(out));
  });
}

} // extern "C"

namespace sdq {

// The Flux attention from q/k/v projections to the merged-heads output,
// written at `out` with row stride `ld_out` elements (a token's heads * 128
// values are contiguous): sdq_flux_attention allocates [B, N, heads * 128];
// the fused single-block op writes the first heads * 128 columns of
// linear2's input.  Returns the output dtype (qkv_a's).
FluxAttnShape flux_attention_shape(sdq_array qkv_a, sdq_array qkv_b, int heads, const StreamImpl *st) {
  const char *op = "flux_attention";
  constexpr int D = 128;
  if (heads <= 0) fail("heads must be positive");
  const int64_t width = int64_t(3) * heads * D;
  FluxAttnShape r;
  sdq_array qkv[2] = {qkv_a, qkv_b};
  for (int i = 0; i < 2; ++i) {
    if (i == 1 && !qkv[1].ctx) break;
    const ArrayImpl *x = float_input(qkv[i], op, i ? "qkv_b" : "qkv_a", st);
    const auto &sh = x->shape;
    if (sh.size() != 3 || sh[2] < width)
      fail("mlx: qkv got " + shape_str(sh) + "; need [batch, tokens, >= 3 * heads * 128]");
    if (i == 0) {
      r.B = sh[0];
      r.dtype = x->dtype;
    } else {
      if (sh[0] != r.B) fail("the two streams must have one batch size");
      if (x->dtype != r.dtype) fail("the two streams must have one dtype");
    }
    r.N += sh[1];
  }
  return r;
}

void flux_attention_into(void *out, int64_t ld_out, sdq_array qkv_a, sdq_array q_norm_a, sdq_array k_norm_a,
                         sdq_array qkv_b, sdq_array q_norm_b, sdq_array k_norm_b, sdq_array pe_cos,
                         sdq_array pe_sin, int heads, float scale, float eps, const StreamImpl *st) {
  const char *op = "flux_attention";
  constexpr int D = 128;
  if (heads <= 0) fail("heads must be positive");
  if (ld_out < int64_t(heads) * D) fail("the output row stride is shorter than heads * 128");
  struct Src {
    ArrayImpl *x = nullptr;
    const ArrayImpl *qn = nullptr, *kn = nullptr;
    int n = 0;
  } src[2];
  sdq_array qkv[2] = {qkv_a, qkv_b}, qn[2] = {q_norm_a, q_norm_b}, kn[2] = {k_norm_a, k_norm_b};
  const FluxAttnShape shp = flux_attention_shape(qkv_a, qkv_b, heads, st);
  for (int i = 0; i < 2; ++i) {
    if (i == 1 && !qkv[1].ctx) break;
    src[i].x = float_input(qkv[i], op, i ? "qkv_b" : "qkv_a", st);
    src[i].n = src[i].x->shape[1];
    if (!qn[i].ctx || !kn[i].ctx) fail("the q and k norm scales are required");
    src[i].qn = norm_param(qn[i], op, "query_norm.scale", D, st);
    src[i].kn = norm_param(kn[i], op, "key_norm.scale", D, st);
  }
  const int B = shp.B;
  const int wdt = src[0].qn->dtype;
  for (int i = 0; i < 2; ++i)
    if (src[i].x && (src[i].qn->dtype != wdt || src[i].kn->dtype != wdt))
      fail("the norm scales must have one dtype");
  const int N = shp.N;
  ArrayImpl *ca = float_input(pe_cos, op, "pe.cos", st);
  ArrayImpl *sa = float_input(pe_sin, op, "pe.sin", st);
  for (const ArrayImpl *p : {ca, sa}) {
    if (p->dtype != SDQ_FLOAT32) fail("the rotary tables must be float32");
    if (int64_t(p->size) != int64_t(N) * (D / 2))
      fail("the rotary tables must hold [1, " + std::to_string(N) + ", 64] values, got " + shape_str(p->shape));
  }
  const int64_t ldt = kern::attention_vt_stride(N);
  auto q = make_array({B, heads, N, D}, SDQ_BFLOAT16, *st);
  auto k = make_array({B, heads, N, D}, SDQ_BFLOAT16, *st);
  auto vt = make_array({B, heads, D, int(ldt)}, SDQ_BFLOAT16, *st);
  kern::FluxPrepSrc pa, pb;
  for (int i = 0; i < 2; ++i) {
    if (!src[i].x) continue;
    kern::FluxPrepSrc &p = i ? pb : pa;
    p.qkv = src[i].x->data();
    p.ld = src[i].x->shape[2];
    p.sb = int64_t(src[i].n) * src[i].x->shape[2];
    p.qn = src[i].qn->data();
    p.kn = src[i].kn->data();
  }
  kern::flux_attention_prep(pa, pb, src[0].x->dtype, wdt, src[0].n, src[1].n, B, heads, eps,
                            static_cast<const float *>(ca->data()), static_cast<const float *>(sa->data()),
                            static_cast<uint16_t *>(q->data()), static_cast<uint16_t *>(k->data()),
                            static_cast<uint16_t *>(vt->data()), ldt, st->stream);
  // merge_heads' layout: token rows of heads * 128 values, row stride ld_out.
  kern::AttnArgs a;
  a.q = static_cast<const uint16_t *>(q->data());
  a.k = static_cast<const uint16_t *>(k->data());
  a.vt = static_cast<const uint16_t *>(vt->data());
  a.o = out;
  a.q_sn = D, a.q_sh = int64_t(N) * D, a.q_sb = int64_t(heads) * N * D;
  a.k_sn = D, a.k_sh = a.q_sh, a.k_sb = a.q_sb;
  a.v_sd = ldt, a.v_sh = int64_t(D) * ldt, a.v_sb = int64_t(heads) * D * ldt;
  a.o_sn = ld_out, a.o_sh = D, a.o_sb = int64_t(N) * ld_out;
  a.B = B, a.H = heads, a.group = 1, a.Nq = N, a.Nk = N, a.D = D;
  a.scale_log2 = scale * 1.4426950408889634f;
  kern::attention(a, shp.dtype, st->stream);
}

} // namespace sdq

extern "C" {

int sdq_flux_attention(sdq_array *res, sdq_array qkv_a, sdq_array q_norm_a, sdq_array k_norm_a, sdq_array qkv_b,
                       sdq_array q_norm_b, sdq_array k_norm_b, sdq_array pe_cos, sdq_array pe_sin, int heads,
                       float scale, float eps, sdq_stream s) {
  SDQ_GUARD("flux_attention", {
    StreamImpl *st = stream_of(s, "flux_attention");
    if (!res) fail("result pointer is NULL");
    constexpr int D = 128;
    const FluxAttnShape shp = flux_attention_shape(qkv_a, qkv_b, heads, st);
    // The output is merge_heads' layout, [batch, tokens, heads * 128].
    auto out = make_array({shp.B, shp.N, heads * D}, shp.dtype, *st);
    flux_attention_into(out->data(), int64_t(heads) * D, qkv_a, q_norm_a, k_norm_a, qkv_b, q_norm_b, k_norm_b,
                        pe_cos, pe_sin, heads, scale, eps, st);
    set_result(res, std::move(out));
  });
}

} // extern "C"
