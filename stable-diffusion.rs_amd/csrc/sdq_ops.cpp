// sdq_ops.cpp -- the op entry points of libsdq's C ABI: quantize, dequantize,
// quantized_matmul and the elementwise ops around them.  Each validates its
// arguments the way the reference's callers expect MLX to (a non-zero status
// and a message, never an abort: mlx.rs:853-863 records MLX aborting on some
// inputs), orders its inputs on the stream, and enqueues HIP kernels.
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "kernels/launch.hpp"
#include "sdq_internal.hpp"

namespace sdq {

// Waits on `s` for the work that produced `a`, when that ran elsewhere, and
// records `s` as a user of a's memory, so that the allocator orders a later
// reuse of the block after this use too.
void order_after(const ArrayImpl *a, const StreamImpl *s) {
  if (a->buf && a->buf->ptr) a->buf->note_reader(s->stream);
  if (!a->stream || a->stream == s->stream || stream_retired(a->stream)) return;
  hipEvent_t ev;
  hip_check(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate");
  hip_check(hipEventRecord(ev, a->stream), "hipEventRecord");
  hip_check(hipStreamWaitEvent(s->stream, ev, 0), "hipStreamWaitEvent");
  hip_check(hipEventDestroy(ev), "hipEventDestroy");
}

void same_device(const ArrayImpl *a, const StreamImpl *s, const char *name) {
  if (a->device != s->device)
    fail(std::string("`") + name + "` lives on device " + std::to_string(a->device) +
         " but the stream is on device " + std::to_string(s->device));
}

namespace {

int opt_or(sdq_optional_int v, int dflt) { return v.has_value ? v.value : dflt; }

void check_mode(const char *mode, sdq_array global_scale) {
  if (mode && std::strcmp(mode, "affine") != 0)
    fail(std::string("Invalid quantization mode '") + mode +
         "'; libsdq implements 'affine' (scale and bias per group)");
  if (global_scale.ctx)
    fail("global_scale applies to the nvfp4 mode only and must be empty for 'affine'");
}

void check_group_bits(int gs, int bits) {
  if (gs != 32 && gs != 64 && gs != 128)
    fail("The requested group size " + std::to_string(gs) +
         " is not supported. The supported group sizes are 32, 64 and 128.");
  if (bits != 2 && bits != 4 && bits != 8)
    fail("The requested number of bits " + std::to_string(bits) +
         " is not supported. The supported bits are 2, 4 and 8.");
}

} // namespace

void matmul_dispatch(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
                     const uint32_t *w, const void *scales, const void *biases,
                     int s_dtype, int64_t M, int64_t N, int64_t K, int gs, int bits,
                     int device, hipStream_t stream, const kern::Epilogue &ep) {
  if (M == 0 || N == 0) return;
  if (ep.pair != 0) {
    if (N % 16 != 0)
      fail("a gated pair's weight has rows in blocks of sixteen (eight gate, eight up), got N = " +
           std::to_string(N));
    if (ep.split != 0 || ep.combine != 0) fail("a gated pair takes no output split or combine stage");
    if (ep.ldy != 0 && ep.ldy < N / 2) fail("the output row stride is shorter than N / 2");
  } else if (ep.split != 0) {
    if (ep.split % 256 != 0 || ep.split <= 0 || ep.split >= N)
      fail("the output split must be a multiple of 256 inside (0, N), got " + std::to_string(ep.split) +
           " for N = " + std::to_string(N));
    if (!ep.y2) fail("the output split needs its second destination");
    if (ep.ldy != 0 && ep.ldy < ep.split) fail("the first destination's row stride is shorter than the split");
    if (ep.ldy2 < N - ep.split) fail("the second destination's row stride is shorter than N - split");
    if (ep.combine != 0) fail("the output split takes no combine stage");
  } else if (ep.ldy != 0 && ep.ldy < N) {
    fail("the output row stride is shorter than N");
  }
  if (gs != 64 && gs != 128)
    fail("the quantized matmul kernels take group size 64 or 128, got " + std::to_string(gs));
  if (bits != 4 && bits != 8)
    fail("the quantized matmul kernels take 4 or 8 bits, got " + std::to_string(bits));
  if (kern::qmv_takes(M, N, K)) {
    const kern::QmvPlan plan = kern::plan_qmv(M, N, K, gs, bits, cu_count(device));
    float *partial = nullptr;
    if (plan.ranges > 1)
      partial = stream_workspace(device, stream, plan.partial_floats) + kWorkspaceHeaderFloats;
    kern::qmv(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K, gs, bits,
              plan, ep, stream, partial);
  } else {
    kern::QmmPlan plan = kern::plan_qmm(M, N, K, bits, cu_count(device));
    kern::SplitWorkspace ws;
    if (plan.dp_tiles < plan.tiles || plan.sk_workers > 0) {
      float *base = stream_workspace(device, stream, plan.partial_floats);
      ws.flags = reinterpret_cast<int *>(base);
      ws.partial = base + kWorkspaceHeaderFloats;
    }
    // The whole epilogue (bias, activation, combine stage) runs in the tile
    // kernel's store, or in the reduction of split tiles.
    kern::qmm(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K, gs, bits,
              plan, ws, ep, stream);
  }
}

namespace {

} // namespace

int cu_count(int device) {
  static std::mutex mu;
  static std::map<int, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(device);
  if (it != cache.end()) return it->second;
  int n = 0;
  hip_check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device),
            "hipDeviceGetAttribute");
  cache[device] = n;
  return n;
}

} // namespace sdq

using namespace sdq;

extern "C" {

int sdq_quantize(sdq_vector_array *res, sdq_array w, sdq_optional_int group_size,
                 sdq_optional_int bits, const char *mode, sdq_array global_scale,
                 sdq_stream s) {
  SDQ_GUARD("quantize", {
    StreamImpl *st = stream_of(s, "quantize");
    if (!res) fail("result pointer is NULL");
    check_mode(mode, global_scale);
    const int gs = opt_or(group_size, 64);
    const int nb = opt_or(bits, 4);
    check_group_bits(gs, nb);
    ArrayImpl *wa = array_of(w, "quantize", "w");
    same_device(wa, st, "w");
    if (wa->shape.size() < 2)
      fail("The matrix to be quantized must have at least 2 dimensions but it has only " +
           std::to_string(wa->shape.size()) + ".");
    if (!is_float_dtype(wa->dtype))
      fail(std::string("Only float32, bfloat16 and float16 matrices can be quantized, got ") +
           dtype_name(wa->dtype));
    const int K = wa->shape.back();
    if (K % gs != 0)
      fail("The last dimension of the matrix needs to be divisible by the quantization "
           "group size " +
           std::to_string(gs) + ". However the provided matrix has shape " +
           shape_str(wa->shape));
    order_after(wa, st);
    std::vector<int> qshape = wa->shape, sshape = wa->shape;
    qshape.back() = int(int64_t(K) * nb / 32);
    sshape.back() = K / gs;
    auto wq = make_array(qshape, SDQ_UINT32, *st);
    auto sc = make_array(sshape, wa->dtype, *st);
    auto bi = make_array(sshape, wa->dtype, *st);
    const int64_t rows = K ? int64_t(wa->size / size_t(K)) : 0;
    kern::quantize(wa->data(), wa->dtype, rows, K, gs, nb,
                   static_cast<uint32_t *>(wq->data()), sc->data(), bi->data(), st->stream);
    std::vector<std::unique_ptr<ArrayImpl>> parts;
    parts.push_back(std::move(wq));
    parts.push_back(std::move(sc));
    parts.push_back(std::move(bi));
    set_vector_result(res, std::move(parts));
  });
}

int sdq_dequantize(sdq_array *res, sdq_array w, sdq_array scales, sdq_array biases,
                   sdq_optional_int group_size, sdq_optional_int bits, const char *mode,
                   sdq_array global_scale, sdq_optional_dtype dtype, sdq_stream s) {
  SDQ_GUARD("dequantize", {
    StreamImpl *st = stream_of(s, "dequantize");
    check_mode(mode, global_scale);
    const int gs = opt_or(group_size, 64);
    const int nb = opt_or(bits, 4);
    check_group_bits(gs, nb);
    ArrayImpl *wa = array_of(w, "dequantize", "w");
    ArrayImpl *sa = array_of(scales, "dequantize", "scales");
    ArrayImpl *ba = array_of(biases, "dequantize", "biases");
    same_device(wa, st, "w");
    same_device(sa, st, "scales");
    same_device(ba, st, "biases");
    if (wa->dtype != SDQ_UINT32)
      fail(std::string("The matrix should be given as a uint32, got ") + dtype_name(wa->dtype));
    if (wa->shape.size() < 2)
      fail("The matrix to be dequantized must have at least 2 dimensions");
    if (sa->shape != ba->shape || sa->dtype != ba->dtype)
      fail("Shape and dtype of scales and biases should match: " + shape_str(sa->shape) + " " +
           dtype_name(sa->dtype) + " vs " + shape_str(ba->shape) + " " + dtype_name(ba->dtype));
    if (!is_float_dtype(sa->dtype))
      fail(std::string("scales must be float32, bfloat16 or float16, got ") + dtype_name(sa->dtype));
    const int64_t K = int64_t(wa->shape.back()) * 32 / nb;
    std::vector<int> lead_w(wa->shape.begin(), wa->shape.end() - 1);
    std::vector<int> lead_s(sa->shape.begin(), sa->shape.end() - 1);
    if (lead_w != lead_s || int64_t(sa->shape.back()) * gs != K)
      fail("Shape of scales and biases does not match the matrix given the quantization "
           "parameters. Provided matrix of shape " +
           shape_str(wa->shape) + " and scales/biases of shape " + shape_str(sa->shape) +
           " with group_size=" + std::to_string(gs) + " and bits=" + std::to_string(nb) + ".");
    int out_dtype = sa->dtype;
    if (dtype.has_value) {
      if (!is_float_dtype(dtype.value))
        fail(std::string("dtype must be float32, bfloat16 or float16, got ") + dtype_name(dtype.value));
      out_dtype = dtype.value;
    }
    order_after(wa, st);
    order_after(sa, st);
    order_after(ba, st);
    std::vector<int> oshape = wa->shape;
    oshape.back() = int(K);
    auto out = make_array(oshape, out_dtype, *st);
    const int64_t rows = K ? int64_t(out->size / size_t(K)) : 0;
    kern::dequantize(static_cast<const uint32_t *>(wa->data()), sa->data(), ba->data(), sa->dtype,
                     rows, K, gs, nb, out->data(), out_dtype, st->stream);
    set_result(res, std::move(out));
  });
}

} // extern "C"

namespace {

// quantized_matmul with an optional output epilogue (bias [N], activation),
// shared by sdq_quantized_matmul and sdq_quantized_linear.
// The quantized weight and activation operands of a linear, checked as
// mlx_quantized_matmul checks them (transpose = true).
struct QOperands {
  ArrayImpl *xa, *wa, *sa, *ba;
  int64_t N, K;
  int gs, nb;
};

QOperands quantized_operands(sdq_array x, sdq_array w, sdq_array scales, sdq_array biases,
                             sdq_optional_int group_size, sdq_optional_int bits, const char *mode,
                             const StreamImpl *st) {
    check_mode(mode, sdq_array{nullptr});
    const int gs = opt_or(group_size, 64);
    const int nb = opt_or(bits, 4);
    check_group_bits(gs, nb);
    ArrayImpl *xa = array_of(x, "quantized_matmul", "x");
    ArrayImpl *wa = array_of(w, "quantized_matmul", "w");
    ArrayImpl *sa = array_of(scales, "quantized_matmul", "scales");
    ArrayImpl *ba = array_of(biases, "quantized_matmul", "biases");
    same_device(xa, st, "x");
    same_device(wa, st, "w");
    same_device(sa, st, "scales");
    same_device(ba, st, "biases");
    if (wa->dtype != SDQ_UINT32)
      fail(std::string("The weight matrix should be uint32, got ") + dtype_name(wa->dtype));
    if (wa->shape.size() != 2)
      fail("The weight matrix must be 2-D [out, in*bits/32], got shape " + shape_str(wa->shape));
    if (!is_float_dtype(xa->dtype))
      fail(std::string("x must be float32, bfloat16 or float16, got ") + dtype_name(xa->dtype));
    if (sa->shape != ba->shape || sa->dtype != ba->dtype || !is_float_dtype(sa->dtype))
      fail("scales and biases must share one float dtype and one shape, got " +
           shape_str(sa->shape) + " " + dtype_name(sa->dtype) + " and " + shape_str(ba->shape) +
           " " + dtype_name(ba->dtype));
    const int64_t N = wa->shape[0];
    const int64_t K = int64_t(wa->shape[1]) * 32 / nb;
    if (sa->shape.size() != 2 || sa->shape[0] != N || int64_t(sa->shape[1]) * gs != K)
      fail("Shape of scales and biases does not match the matrix given the quantization "
           "parameters. Provided matrix of shape " +
           shape_str(wa->shape) + " and scales/biases of shape " + shape_str(sa->shape) +
           " with group_size=" + std::to_string(gs) + " and bits=" + std::to_string(nb) + ".");
    if (xa->shape.empty() || xa->shape.back() != K)
      fail("Last dimension of first input with shape " + shape_str(xa->shape) +
           " must match the dequantized weight's input width " + std::to_string(K) +
           " (weight " + shape_str(wa->shape) + ", bits=" + std::to_string(nb) + ")");
    return QOperands{xa, wa, sa, ba, N, K, gs, nb};
}

// The bias of a linear: a float array of N values, or none.
ArrayImpl *linear_bias(sdq_array bias, int64_t N, const StreamImpl *st, kern::Epilogue &ep) {
    if (!bias.ctx) return nullptr;
    ArrayImpl *bb = array_of(bias, "quantized_linear", "bias");
    same_device(bb, st, "bias");
    if (!is_float_dtype(bb->dtype) || bb->size != size_t(N) || (!bb->shape.empty() && bb->shape.back() != N))
      fail("bias must be a float array of shape [" + std::to_string(N) + "], got " +
           shape_str(bb->shape) + " " + dtype_name(bb->dtype));
    ep.bias = bb->data();
    ep.bias_dtype = bb->dtype;
    return bb;
}

void quantized_matmul_impl(sdq_array *res, sdq_array x, sdq_array w, sdq_array scales,
                           sdq_array biases, bool transpose, sdq_optional_int group_size,
                           sdq_optional_int bits, const char *mode, sdq_stream s,
                           sdq_array bias, int activation, sdq_array residual = sdq_array{nullptr},
                           sdq_array gate = sdq_array{nullptr}, int combine = SDQ_COMBINE_NONE,
                           bool pair = false) {
    StreamImpl *st = stream_of(s, "quantized_matmul");
    if (!transpose)
      fail("transpose=false (x @ W with W quantized along its output axis) is not "
           "implemented; the diffusers [out, in] layout uses transpose=true");
    const QOperands q = quantized_operands(x, w, scales, biases, group_size, bits, mode, st);
    ArrayImpl *xa = q.xa, *wa = q.wa, *sa = q.sa, *ba = q.ba;
    const int64_t N = q.N, K = q.K;
    const int gs = q.gs, nb = q.nb;
    kern::Epilogue ep;
    ArrayImpl *bb = linear_bias(bias, N, st, ep);
    if (activation != SDQ_ACT_NONE && activation != SDQ_ACT_GELU_APPROX)
      fail("activation must be SDQ_ACT_NONE or SDQ_ACT_GELU_APPROX, got " + std::to_string(activation));
    ep.act = activation;
    ArrayImpl *ra = nullptr, *ga = nullptr;
    if (combine != SDQ_COMBINE_NONE) {
      if (combine != SDQ_COMBINE_GATED_RESIDUAL && combine != SDQ_COMBINE_PRODUCT)
        fail("combine must be SDQ_COMBINE_NONE, SDQ_COMBINE_GATED_RESIDUAL or SDQ_COMBINE_PRODUCT, got " +
             std::to_string(combine));
      if (!residual.ctx) fail("combine needs the residual (or product) operand");
      ra = array_of(residual, "quantized_linear", "residual");
      same_device(ra, st, "residual");
      std::vector<int> want = xa->shape;
      want.back() = int(N);
      if (!is_float_dtype(ra->dtype) || ra->shape != want)
        fail("residual must be a float array of the output's shape " + shape_str(want) + ", got " +
             shape_str(ra->shape) + " " + dtype_name(ra->dtype));
      ep.res = ra->data();
      ep.res_dtype = ra->dtype;
      ep.ld_res = N;
      if (gate.ctx) {
        if (combine != SDQ_COMBINE_GATED_RESIDUAL) fail("a gate applies to SDQ_COMBINE_GATED_RESIDUAL only");
        ga = array_of(gate, "quantized_linear", "gate");
        same_device(ga, st, "gate");
        if (!is_float_dtype(ga->dtype) || ga->size != size_t(N) || (!ga->shape.empty() && ga->shape.back() != N))
          fail("gate must be a float array of N = " + std::to_string(N) + " values, got " +
               shape_str(ga->shape) + " " + dtype_name(ga->dtype));
        ep.gate = ga->data();
        ep.gate_dtype = ga->dtype;
      }
    } else if (residual.ctx || gate.ctx) {
      fail("a residual or gate was given without a combine mode");
    }
    ep.combine = combine;
    if (pair) {
      if (N % 16 != 0)
        fail("a gated pair's weight has rows in blocks of sixteen (eight gate, eight up; sdq_pair_rows), "
             "got " + std::to_string(N) + " rows");
      ep.pair = 1;
    }
    const int out_dtype = promote_float(xa->dtype, sa->dtype);
    if (bb) order_after(bb, st);
    if (ra) order_after(ra, st);
    if (ga) order_after(ga, st);
    order_after(xa, st);
    order_after(wa, st);
    order_after(sa, st);
    order_after(ba, st);
    std::vector<int> oshape = xa->shape;
    oshape.back() = int(pair ? N / 2 : N);
    auto out = make_array(oshape, out_dtype, *st);
    const int64_t M = K ? int64_t(xa->size / size_t(K)) : 0;
    matmul_dispatch(out->data(), out_dtype, xa->data(), xa->dtype, K,
                    static_cast<const uint32_t *>(wa->data()), sa->data(), ba->data(), sa->dtype,
                    M, N, K, gs, nb, st->device, st->stream, ep);
    set_result(res, std::move(out));
}

} // namespace

extern "C" {

int sdq_quantized_matmul(sdq_array *res, sdq_array x, sdq_array w, sdq_array scales,
                         sdq_array biases, bool transpose, sdq_optional_int group_size,
                         sdq_optional_int bits, const char *mode, sdq_stream s) {
  SDQ_GUARD("quantized_matmul", {
    quantized_matmul_impl(res, x, w, scales, biases, transpose, group_size, bits, mode, s,
                          sdq_array{nullptr}, SDQ_ACT_NONE);
  });
}

int sdq_quantized_linear(sdq_array *res, sdq_array x, sdq_array w, sdq_array scales,
                         sdq_array biases, sdq_array bias, int activation,
                         sdq_optional_int group_size, sdq_optional_int bits, const char *mode,
                         sdq_stream s) {
  SDQ_GUARD("quantized_linear", {
    quantized_matmul_impl(res, x, w, scales, biases, true, group_size, bits, mode, s, bias,
                          activation);
  });
}

int sdq_quantized_linear_combine(sdq_array *res, sdq_array x, sdq_array w, sdq_array scales,
                                 sdq_array biases, sdq_array bias, int activation,
                                 sdq_array residual, sdq_array gate, int combine,
                                 sdq_optional_int group_size, sdq_optional_int bits,
                                 const char *mode, sdq_stream s) {
  SDQ_GUARD("quantized_linear_combine", {
    quantized_matmul_impl(res, x, w, scales, biases, true, group_size, bits, mode, s, bias,
                          activation, residual, gate, combine);
  });
}



int sdq_quantized_linear_gated(sdq_array *res, sdq_array x, sdq_array w, sdq_array scales,
                               sdq_array biases, sdq_array bias, int activation,
                               sdq_optional_int group_size, sdq_optional_int bits, const char *mode,
                               sdq_stream s) {
  SDQ_GUARD("quantized_linear_gated", {
    quantized_matmul_impl(res, x, w, scales, biases, true, group_size, bits, mode, s, bias,
                          activation, sdq_array{nullptr}, sdq_array{nullptr}, SDQ_COMBINE_NONE, true);
  });
}

int sdq_pair_rows(sdq_array *res, sdq_array gate, sdq_array up, sdq_stream s) {
  SDQ_GUARD("pair_rows", {
    StreamImpl *st = stream_of(s, "pair_rows");
    if (!res) fail("result pointer is NULL");
    ArrayImpl *ga = array_of(gate, "pair_rows", "gate");
    ArrayImpl *ua = array_of(up, "pair_rows", "up");
    same_device(ga, st, "gate");
    same_device(ua, st, "up");
    if (ga->shape != ua->shape || ga->dtype != ua->dtype)
      fail("gate and up must share one shape and dtype, got " + shape_str(ga->shape) + " " +
           dtype_name(ga->dtype) + " and " + shape_str(ua->shape) + " " + dtype_name(ua->dtype));
    if (ga->shape.empty() || ga->shape[0] % 8 != 0 || ga->shape[0] <= 0)
      fail("pair_rows takes arrays whose first dimension is a positive multiple of 8, got " +
           shape_str(ga->shape));
    const int64_t rows = ga->shape[0];
    const size_t row_bytes = ga->nbytes() / size_t(rows);
    std::vector<int> oshape = ga->shape;
    oshape[0] = int(2 * rows);
    order_after(ga, st);
    order_after(ua, st);
    auto out = make_array(oshape, ga->dtype, *st);
    // Blocks of eight rows: gate's block b to result rows 16 b.., up's to
    // 16 b + 8.. -- two strided copies.
    if (row_bytes > 0) {
      unsigned char *dst = static_cast<unsigned char *>(out->data());
      const size_t blk = 8 * row_bytes;
      hip_check(hipMemcpy2DAsync(dst, 2 * blk, ga->data(), blk, blk, size_t(rows / 8),
                                 hipMemcpyDeviceToDevice, st->stream),
                "hipMemcpy2DAsync");
      hip_check(hipMemcpy2DAsync(dst + blk, 2 * blk, ua->data(), blk, blk, size_t(rows / 8),
                                 hipMemcpyDeviceToDevice, st->stream),
                "hipMemcpy2DAsync");
    }
    set_result(res, std::move(out));
  });
}

int sdq_quantized_linear_gated_raw(void *y, int64_t ldy, int y_dtype, const void *x, int x_dtype,
                                   int64_t ldx, const uint32_t *w, const void *scales, const void *biases,
                                   int s_dtype, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                   const void *bias, int bias_dtype, int activation, void *hip_stream) {
  SDQ_GUARD("quantized_linear_gated_raw", {
    if (M < 0 || N < 0 || K <= 0) fail("M, N must be >= 0 and K > 0");
    if (!is_float_dtype(x_dtype) || !is_float_dtype(s_dtype) || !is_float_dtype(y_dtype))
      fail("dtypes must be float32, bfloat16 or float16");
    if (bias && !is_float_dtype(bias_dtype))
      fail("bias dtype must be float32, bfloat16 or float16");
    if (activation != SDQ_ACT_NONE && activation != SDQ_ACT_GELU_APPROX)
      fail("activation must be SDQ_ACT_NONE or SDQ_ACT_GELU_APPROX, got " + std::to_string(activation));
    check_group_bits(group_size, bits);
    if (K % group_size != 0) fail("K must be a multiple of group_size");
    if (N % 16 != 0) fail("N (the paired weight's rows) must be a multiple of 16, got " + std::to_string(N));
    if (ldy < 0) fail("negative output row stride");
    if (M > 0 && N > 0 && (!y || !x || !w || !scales || !biases)) fail("NULL pointer argument");
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    kern::Epilogue ep;
    ep.bias = bias;
    ep.bias_dtype = bias ? bias_dtype : 0;
    ep.act = activation;
    ep.ldy = ldy;
    ep.pair = 1;
    if (!kern::epilogue_ok(ep)) fail("bad epilogue");
    matmul_dispatch(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K,
                    group_size, bits, device, static_cast<hipStream_t>(hip_stream), ep);
  });
}

int sdq_quantized_matmul_raw(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
                             const uint32_t *w, const void *scales, const void *biases,
                             int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
                             int bits, void *hip_stream) {
  SDQ_GUARD("quantized_matmul_raw", {
    if (M < 0 || N < 0 || K <= 0) fail("M, N must be >= 0 and K > 0");
    if (!is_float_dtype(x_dtype) || !is_float_dtype(s_dtype) || !is_float_dtype(y_dtype))
      fail("dtypes must be float32, bfloat16 or float16");
    check_group_bits(group_size, bits);
    if (K % group_size != 0) fail("K must be a multiple of group_size");
    if (M > 0 && N > 0 && (!y || !x || !w || !scales || !biases)) fail("NULL pointer argument");
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    matmul_dispatch(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K,
                    group_size, bits, device, static_cast<hipStream_t>(hip_stream), kern::Epilogue{});
  });
}

int sdq_quantized_matmul_epilogue_raw(void *y, int y_dtype, const void *x, int x_dtype,
                                      int64_t ldx, const uint32_t *w, const void *scales,
                                      const void *biases, int s_dtype, int64_t M, int64_t N,
                                      int64_t K, int group_size, int bits, const void *bias,
                                      int bias_dtype, int activation, void *hip_stream) {
  SDQ_GUARD("quantized_matmul_epilogue_raw", {
    if (M < 0 || N < 0 || K <= 0) fail("M, N must be >= 0 and K > 0");
    if (!is_float_dtype(x_dtype) || !is_float_dtype(s_dtype) || !is_float_dtype(y_dtype))
      fail("dtypes must be float32, bfloat16 or float16");
    if (bias && !is_float_dtype(bias_dtype))
      fail("bias dtype must be float32, bfloat16 or float16");
    if (activation != SDQ_ACT_NONE && activation != SDQ_ACT_GELU_APPROX)
      fail("activation must be SDQ_ACT_NONE or SDQ_ACT_GELU_APPROX, got " + std::to_string(activation));
    check_group_bits(group_size, bits);
    if (K % group_size != 0) fail("K must be a multiple of group_size");
    if (M > 0 && N > 0 && (!y || !x || !w || !scales || !biases)) fail("NULL pointer argument");
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    kern::Epilogue ep;
    ep.bias = bias;
    ep.bias_dtype = bias ? bias_dtype : 0;
    ep.act = activation;
    if (!kern::epilogue_ok(ep)) fail("bad epilogue");
    matmul_dispatch(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K,
                    group_size, bits, device, static_cast<hipStream_t>(hip_stream), ep);
  });
}

int sdq_quantized_linear_split_raw(void *y, int64_t ldy, int activation, void *y2, int64_t ldy2,
                                   int activation2, int64_t split, int y_dtype, const void *x, int x_dtype,
                                   int64_t ldx, const uint32_t *w, const void *scales, const void *biases,
                                   int s_dtype, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                                   const void *bias, int bias_dtype, void *hip_stream) {
  SDQ_GUARD("quantized_linear_split_raw", {
    if (M < 0 || N < 0 || K <= 0) fail("M, N must be >= 0 and K > 0");
    if (!is_float_dtype(x_dtype) || !is_float_dtype(s_dtype) || !is_float_dtype(y_dtype))
      fail("dtypes must be float32, bfloat16 or float16");
    if (bias && !is_float_dtype(bias_dtype))
      fail("bias dtype must be float32, bfloat16 or float16");
    for (int a : {activation, activation2})
      if (a != SDQ_ACT_NONE && a != SDQ_ACT_GELU_APPROX)
        fail("activation must be SDQ_ACT_NONE or SDQ_ACT_GELU_APPROX, got " + std::to_string(a));
    check_group_bits(group_size, bits);
    if (K % group_size != 0) fail("K must be a multiple of group_size");
    if (M > 0 && N > 0 && (!y || !y2 || !x || !w || !scales || !biases)) fail("NULL pointer argument");
    if (split <= 0) fail("split must be positive (sdq_quantized_matmul_epilogue_raw has no split)");
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    kern::Epilogue ep;
    ep.bias = bias;
    ep.bias_dtype = bias ? bias_dtype : 0;
    ep.act = activation;
    ep.ldy = ldy;
    ep.split = split;
    ep.y2 = y2;
    ep.ldy2 = ldy2;
    ep.act2 = activation2;
    if (!kern::epilogue_ok(ep)) fail("bad epilogue: split must be a multiple of 256, row strides positive");
    matmul_dispatch(y, y_dtype, x, x_dtype, ldx, w, scales, biases, s_dtype, M, N, K,
                    group_size, bits, device, static_cast<hipStream_t>(hip_stream), ep);
  });
}

int sdq_flux_single_linear1_attention(sdq_array *res, sdq_array x, sdq_array w, sdq_array scales,
                                      sdq_array biases, sdq_array bias, sdq_optional_int group_size,
                                      sdq_optional_int bits, const char *mode, sdq_array q_norm,
                                      sdq_array k_norm, sdq_array pe_cos, sdq_array pe_sin, int heads,
                                      float scale, float eps, sdq_stream s) {
  SDQ_GUARD("flux_single_linear1_attention", {
    StreamImpl *st = stream_of(s, "flux_single_linear1_attention");
    if (!res) fail("result pointer is NULL");
    const QOperands q = quantized_operands(x, w, scales, biases, group_size, bits, mode, st);
    if (q.xa->shape.size() != 3) fail("x must be [batch, tokens, hidden], got " + shape_str(q.xa->shape));
    if (heads <= 0) fail("heads must be positive");
    const int64_t h = int64_t(heads) * 128;
    const int64_t qkv_w = 3 * h, mlp = q.N - qkv_w;
    if (mlp <= 0) fail("linear1 must have more than 3 * heads * 128 outputs (q, k, v, then the MLP)");
    if (qkv_w % 256 != 0) fail("3 * heads * 128 must be a multiple of 256 (an even head count)");
    kern::Epilogue ep;
    ArrayImpl *bb = linear_bias(bias, q.N, st, ep);
    const int out_dtype = promote_float(q.xa->dtype, q.sa->dtype);
    const int B = q.xa->shape[0], T = q.xa->shape[1];
    if (bb) order_after(bb, st);
    order_after(q.xa, st);
    order_after(q.wa, st);
    order_after(q.sa, st);
    order_after(q.ba, st);
    // linear1's q/k/v columns go to a buffer of their own; its MLP columns,
    // through GELU, to linear2's input after the attention's columns.
    auto qkv = make_array({B, T, int(qkv_w)}, out_dtype, *st);
    auto joined = make_array({B, T, int(h + mlp)}, out_dtype, *st);
    ep.act = SDQ_ACT_NONE;
    ep.ldy = qkv_w;
    ep.split = qkv_w;
    ep.y2 = static_cast<unsigned char *>(joined->data()) + size_t(h) * dtype_size(out_dtype);
    ep.ldy2 = h + mlp;
    ep.act2 = SDQ_ACT_GELU_APPROX;
    const int64_t M = int64_t(B) * T;
    matmul_dispatch(qkv->data(), out_dtype, q.xa->data(), q.xa->dtype, q.K,
                    static_cast<const uint32_t *>(q.wa->data()), q.sa->data(), q.ba->data(), q.sa->dtype,
                    M, q.N, q.K, q.gs, q.nb, st->device, st->stream, ep);
    flux_attention_into(joined->data(), h + mlp, sdq_array{qkv.get()}, q_norm, k_norm, sdq_array{nullptr},
                        sdq_array{nullptr}, sdq_array{nullptr}, pe_cos, pe_sin, heads, scale, eps, st);
    set_result(res, std::move(joined));
  });
}

int sdq_gelu_approx_raw(void *out, const void *in, int dtype, int64_t n, void *hip_stream) {
  SDQ_GUARD("gelu_approx_raw", {
    if (!is_float_dtype(dtype)) fail("dtype must be float32, bfloat16 or float16");
    if (n < 0) fail("negative element count");
    if (n > 0 && (!out || !in)) fail("NULL pointer argument");
    kern::gelu_approx(in, dtype, out, n, static_cast<hipStream_t>(hip_stream));
  });
}

void *sdq_array_device_ptr(sdq_array arr) {
  auto *a = static_cast<ArrayImpl *>(arr.ctx);
  return a ? a->data() : nullptr;
}

int sdq_add(sdq_array *res, sdq_array a, sdq_array b, sdq_stream s) {
  SDQ_GUARD("add", {
    StreamImpl *st = stream_of(s, "add");
    ArrayImpl *aa = array_of(a, "add", "a");
    ArrayImpl *bb = array_of(b, "add", "b");
    same_device(aa, st, "a");
    same_device(bb, st, "b");
    if (!is_float_dtype(aa->dtype) || !is_float_dtype(bb->dtype))
      fail("add takes float32, bfloat16 or float16 arrays");
    const bool same = aa->shape == bb->shape;
    const bool bias = bb->shape.size() == 1 && !aa->shape.empty() &&
                      bb->shape[0] == aa->shape.back();
    if (!same && !bias)
      fail("Shapes " + shape_str(aa->shape) + " and " + shape_str(bb->shape) +
           " cannot be broadcast (libsdq adds equal shapes or a bias along the last axis)");
    order_after(aa, st);
    order_after(bb, st);
    const int od = promote_float(aa->dtype, bb->dtype);
    auto out = make_array(aa->shape, od, *st);
    kern::add(aa->data(), aa->dtype, bb->data(), bb->dtype, out->data(), od,
              int64_t(aa->size), int64_t(bb->size), st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_multiply(sdq_array *res, sdq_array a, sdq_array b, sdq_stream s) {
  SDQ_GUARD("multiply", {
    StreamImpl *st = stream_of(s, "multiply");
    ArrayImpl *aa = array_of(a, "multiply", "a");
    ArrayImpl *bb = array_of(b, "multiply", "b");
    same_device(aa, st, "a");
    same_device(bb, st, "b");
    if (!is_float_dtype(aa->dtype) || !is_float_dtype(bb->dtype))
      fail("multiply takes float32, bfloat16 or float16 arrays");
    if (aa->shape != bb->shape)
      fail("Shapes " + shape_str(aa->shape) + " and " + shape_str(bb->shape) +
           " must be equal");
    order_after(aa, st);
    order_after(bb, st);
    const int od = promote_float(aa->dtype, bb->dtype);
    auto out = make_array(aa->shape, od, *st);
    kern::multiply(aa->data(), aa->dtype, bb->data(), bb->dtype, out->data(), od,
                   int64_t(aa->size), st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_astype(sdq_array *res, sdq_array a, sdq_dtype dtype, sdq_stream s) {
  SDQ_GUARD("astype", {
    StreamImpl *st = stream_of(s, "astype");
    ArrayImpl *aa = array_of(a, "astype", "a");
    same_device(aa, st, "a");
    order_after(aa, st);
    auto out = make_array(aa->shape, dtype, *st);
    if (aa->dtype == int(dtype)) {
      if (out->nbytes())
        hip_check(hipMemcpyAsync(out->data(), aa->data(), out->nbytes(),
                                 hipMemcpyDeviceToDevice, st->stream),
                  "hipMemcpyAsync");
    } else {
      if (!is_float_dtype(aa->dtype) || !is_float_dtype(dtype))
        fail(std::string("astype converts between float32, bfloat16 and float16, not ") +
             dtype_name(aa->dtype) + " -> " + dtype_name(dtype));
      kern::astype(aa->data(), aa->dtype, out->data(), dtype, int64_t(aa->size), st->stream);
    }
    set_result(res, std::move(out));
  });
}

int sdq_contiguous(sdq_array *res, sdq_array a, bool allow_col_major, sdq_stream s) {
  (void)allow_col_major;
  SDQ_GUARD("contiguous", {
    StreamImpl *st = stream_of(s, "contiguous");
    ArrayImpl *aa = array_of(a, "contiguous", "a");
    same_device(aa, st, "a");
    order_after(aa, st);
    auto out = make_array(aa->shape, aa->dtype, *st);
    if (out->nbytes())
      hip_check(hipMemcpyAsync(out->data(), aa->data(), out->nbytes(), hipMemcpyDeviceToDevice,
                               st->stream),
                "hipMemcpyAsync");
    set_result(res, std::move(out));
  });
}

int sdq_matmul_nt(sdq_array *res, sdq_array a, sdq_array b, sdq_stream s) {
  SDQ_GUARD("matmul", {
    StreamImpl *st = stream_of(s, "matmul");
    ArrayImpl *aa = array_of(a, "matmul", "a");
    ArrayImpl *bb = array_of(b, "matmul", "b");
    same_device(aa, st, "a");
    same_device(bb, st, "b");
    if (!is_float_dtype(aa->dtype) || !is_float_dtype(bb->dtype))
      fail("matmul takes float32, bfloat16 or float16 arrays");
    if (bb->shape.size() != 2 || aa->shape.empty() || aa->shape.back() != bb->shape[1])
      fail("Shapes " + shape_str(aa->shape) + " and " + shape_str(bb->shape) +
           " do not contract: a is [..., K] and b is [N, K]");
    order_after(aa, st);
    order_after(bb, st);
    const int64_t K = bb->shape[1];
    const int64_t N = bb->shape[0];
    std::vector<int> oshape = aa->shape;
    oshape.back() = int(N);
    const int od = promote_float(aa->dtype, bb->dtype);
    auto out = make_array(oshape, od, *st);
    const int64_t M = K ? int64_t(aa->size / size_t(K)) : 0;
    if (K == 0) fail("matmul over an empty contraction axis");
    kern::matmul_nt(aa->data(), aa->dtype, bb->data(), bb->dtype, out->data(), M, N, K,
                    st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_gelu_approx(sdq_array *res, sdq_array a, sdq_stream s) {
  SDQ_GUARD("gelu_approx", {
    StreamImpl *st = stream_of(s, "gelu_approx");
    ArrayImpl *aa = array_of(a, "gelu_approx", "a");
    same_device(aa, st, "a");
    if (!is_float_dtype(aa->dtype)) fail("gelu_approx takes a float array");
    order_after(aa, st);
    auto out = make_array(aa->shape, aa->dtype, *st);
    kern::gelu_approx(aa->data(), aa->dtype, out->data(), int64_t(aa->size), st->stream);
    set_result(res, std::move(out));
  });
}

} // extern "C"

// ---- GGUF tensors (mlx_gguf.rs:235-276; quantized.rs:181-258) ----------------

namespace {

// The shape of a GGUF tensor as the caller read it from the file's directory
// (already row-major, mlx_gguf.rs:97-104, 208), checked against its raw bytes.
struct GgufTensor {
  std::vector<int> shape;
  int64_t n = 1;
  int64_t raw_bytes = 0;
};

GgufTensor gguf_tensor(const ArrayImpl *raw, int ggml_type, const int *shape, int ndim) {
  int64_t per = 0, bytes = 0;
  if (!kern::gguf_block(ggml_type, &per, &bytes))
    fail("gguf: type " + std::to_string(ggml_type) +
         " is not one this project's checkpoints use; the supported set is F32, F16, BF16, "
         "Q4_0, Q8_0, Q4_K, Q5_K, Q6_K");
  if (raw->dtype != SDQ_UINT8) fail("gguf: `raw` must be a uint8 array of the tensor's bytes");
  if (ndim < 0 || (ndim > 0 && !shape)) fail("gguf: invalid shape");
  GgufTensor t;
  for (int i = 0; i < ndim; ++i) {
    if (shape[i] < 0) fail("gguf: negative dimension in shape " + shape_str(std::vector<int>(shape, shape + ndim)));
    t.shape.push_back(shape[i]);
    t.n *= shape[i];
  }
  if (t.n % per != 0)
    fail("gguf: the tensor has " + std::to_string(t.n) + " elements, not a multiple of " +
         std::to_string(per));
  t.raw_bytes = t.n / per * bytes;
  if (int64_t(raw->nbytes()) != t.raw_bytes)
    fail("gguf: " + std::to_string(raw->nbytes()) + " raw bytes given, a tensor of shape " +
         shape_str(t.shape) + " needs " + std::to_string(t.raw_bytes));
  return t;
}

} // namespace

extern "C" {

int sdq_gguf_dequantize(sdq_array *res, sdq_array raw, int ggml_type, const int *shape, int ndim,
                        sdq_stream s) {
  SDQ_GUARD("gguf_dequantize", {
    StreamImpl *st = stream_of(s, "gguf_dequantize");
    if (!res) fail("result pointer is NULL");
    ArrayImpl *ra = array_of(raw, "gguf_dequantize", "raw");
    same_device(ra, st, "raw");
    const GgufTensor t = gguf_tensor(ra, ggml_type, shape, ndim);
    order_after(ra, st);
    auto out = make_array(t.shape, SDQ_FLOAT32, *st);
    kern::gguf_dequantize(static_cast<const uint8_t *>(ra->data()), ggml_type, t.n, t.raw_bytes,
                          static_cast<float *>(out->data()), st->stream);
    set_result(res, std::move(out));
  });
}

int sdq_gguf_quantize(sdq_vector_array *res, sdq_array raw, int ggml_type, const int *shape,
                      int ndim, sdq_optional_int group_size, sdq_optional_int bits,
                      sdq_stream s) {
  SDQ_GUARD("gguf_quantize", {
    StreamImpl *st = stream_of(s, "gguf_quantize");
    if (!res) fail("result pointer is NULL");
    const int gs = opt_or(group_size, 64);
    const int nb = opt_or(bits, 4);
    check_group_bits(gs, nb);
    ArrayImpl *ra = array_of(raw, "gguf_quantize", "raw");
    same_device(ra, st, "raw");
    const GgufTensor t = gguf_tensor(ra, ggml_type, shape, ndim);
    if (t.shape.size() < 2)
      fail("The matrix to be quantized must have at least 2 dimensions but it has only " +
           std::to_string(t.shape.size()) + ".");
    const int K = t.shape.back();
    if (K % gs != 0)
      fail("The last dimension of the matrix needs to be divisible by the quantization "
           "group size " +
           std::to_string(gs) + ". However the provided matrix has shape " + shape_str(t.shape));
    order_after(ra, st);
    std::vector<int> qshape = t.shape, sshape = t.shape;
    qshape.back() = int(int64_t(K) * nb / 32);
    sshape.back() = K / gs;
    auto wq = make_array(qshape, SDQ_UINT32, *st);
    auto sc = make_array(sshape, SDQ_FLOAT32, *st);
    auto bi = make_array(sshape, SDQ_FLOAT32, *st);
    const int64_t rows = K ? t.n / K : 0;
    kern::gguf_quantize(static_cast<const uint8_t *>(ra->data()), ggml_type, rows, K, t.raw_bytes, gs,
                        nb, static_cast<uint32_t *>(wq->data()), static_cast<float *>(sc->data()),
                        static_cast<float *>(bi->data()), st->stream);
    std::vector<std::unique_ptr<ArrayImpl>> parts;
    parts.push_back(std::move(wq));
    parts.push_back(std::move(sc));
    parts.push_back(std::move(bi));
    set_vector_result(res, std::move(parts));
  });
}

} // extern "C"
