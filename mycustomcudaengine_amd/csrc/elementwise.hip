// Bandwidth-bound fused ops: RMSNorm, SwiGLU, paged KV store, in-place RoPE.
//
// All four are HBM-bound streaming kernels.  Each uses 16-byte global accesses
// (8 x 16-bit values per lane) where the row length and alignment allow, and a
// scalar fallback otherwise; fp32 arithmetic, one rounding to storage type.
#include "mce_common.h"

namespace mce {

// =========================================================================
// RMSNorm  (reference: csrc/kernels/rmsnorm.cu:35-108)
//
// One wave per row, a workgroup of its own (one-wave workgroups spread the
// rows over more CUs than four-row ones: 16384 x 4096 40.1 -> 38.6 us, 4096 x
// 3072 9.1 -> 6.7 us on MI355X, with the stores below; 20-call graphs).  The row stays in
// registers between the sum-of-squares pass and the scaling pass, so every
// input byte is read once: VPT 16-byte vectors per lane cover rows up to
// 512 * VPT elements.  The output goes out with non-temporal stores (it is
// not read again by this kernel; plain stores measured 2-28% slower).  Rows
// longer than 8192 elements (or not 16-byte aligned) take the two-pass
// kernel, whose second read hits L2.
// =========================================================================
template <class T, int VPT>
__global__ __launch_bounds__(64) void rmsnorm_vec_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ w,
    uint16_t *__restrict__ y, int64_t rows, int hidden, int64_t in_stride,
    int64_t out_stride, float eps) {
  // one row per workgroup (a loop over rows let the compiler wait for the
  // first of a row's loads before issuing the rest: 38.6 -> 40.4 us at
  // 16384 x 4096)
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int nvec = hidden >> 3;  // 8 elements per 16-byte vector
  const u32x4 *xr = reinterpret_cast<const u32x4 *>(x + row * in_stride);
  const u32x4 *wr = reinterpret_cast<const u32x4 *>(w);
  u32x4 v[VPT], wv[VPT];
  // Every load is unconditional (chunks past the row re-read its last chunk
  // and are zeroed by a select): a load under a per-lane condition becomes an
  // exec-masked branch that waits for the loads before it, which kept one
  // 16-byte load per wave in flight and halved the bandwidth.  A zeroed chunk
  // adds fma(0, 0, ss) = ss, so the sum is the one over the row's chunks.
  // The weight loads go out right behind the row loads, ahead of the
  // reduction: the scheduling barrier keeps the scheduler from sinking them
  // past it (one more round trip per row).
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = lane + i * 64;
    v[i] = xr[idx < nvec ? idx : nvec - 1];
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = lane + i * 64;
    wv[i] = wr[idx < nvec ? idx : nvec - 1];
  }
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = lane + i * 64;
    v[i] = idx < nvec ? v[i] : u32x4{0, 0, 0, 0};
    ss = sumsq8<T>(v[i], ss);
  }
  ss = wave_sum(ss);
  const float inv = rms_inv(ss, hidden, eps);
  // outputs computed unconditionally, then stored where in the row (the
  // empty asm takes each one in registers, so that neither the computation
  // nor its weight load sinks into the store's branch: one more round trip)
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    v[i] = rms_scale8<T>(v[i], wv[i], inv);
    asm volatile("" : "+v"(v[i]));
  }
  u32x4 *yr = reinterpret_cast<u32x4 *>(y + row * out_stride);
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = lane + i * 64;
    if (idx < nvec) __builtin_nontemporal_store(v[i], yr + idx);
  }
}

template <class T>
__global__ __launch_bounds__(256) void rmsnorm_generic_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ w,
    uint16_t *__restrict__ y, int64_t rows, int hidden, int64_t in_stride,
    int64_t out_stride, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t *xr = x + row * in_stride;
  float ss = 0.f;
  for (int i = lane; i < hidden; i += 64) {
    float a = T::lo(xr[i]);
    ss += a * a;
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
  uint16_t *yr = y + row * out_stride;
  for (int i = lane; i < hidden; i += 64)
    yr[i] = T::from_float(T::lo(xr[i]) * (inv * T::lo(w[i])));
}

template <class T>
static int rmsnorm_launch(const void *input, const void *weight, void *output,
                          int64_t rows, int64_t hidden, int64_t in_stride,
                          int64_t out_stride, float eps, hipStream_t st) {
  const uint16_t *x = (const uint16_t *)input;
  const uint16_t *w = (const uint16_t *)weight;
  uint16_t *y = (uint16_t *)output;
  const bool vec = hidden % 8 == 0 && in_stride % 8 == 0 &&
                   out_stride % 8 == 0 && aligned16(x) && aligned16(w) &&
                   aligned16(y);
  const int nvec = (int)(hidden / 8);
  int h = (int)hidden;
  // vector kernels: one 64-lane workgroup per row (the entry point keeps
  // rows below 2^31)
  const dim3 vgrid((unsigned)rows), vblock(64);
  if (vec && nvec <= 64)
    rmsnorm_vec_kernel<T, 1><<<vgrid, vblock, 0, st>>>(x, w, y, rows, h, in_stride, out_stride, eps);
  else if (vec && nvec <= 128)
    rmsnorm_vec_kernel<T, 2><<<vgrid, vblock, 0, st>>>(x, w, y, rows, h, in_stride, out_stride, eps);
  else if (vec && nvec <= 256)
    rmsnorm_vec_kernel<T, 4><<<vgrid, vblock, 0, st>>>(x, w, y, rows, h, in_stride, out_stride, eps);
  else if (vec && nvec <= 384)
    rmsnorm_vec_kernel<T, 6><<<vgrid, vblock, 0, st>>>(x, w, y, rows, h, in_stride, out_stride, eps);
  else if (vec && nvec <= 512)
    rmsnorm_vec_kernel<T, 8><<<vgrid, vblock, 0, st>>>(x, w, y, rows, h, in_stride, out_stride, eps);
  else if (vec && nvec <= 1024)
    rmsnorm_vec_kernel<T, 16><<<vgrid, vblock, 0, st>>>(x, w, y, rows, h, in_stride, out_stride, eps);
  else
    rmsnorm_generic_kernel<T><<<dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st>>>(
        x, w, y, rows, h, in_stride, out_stride, eps);
  return check_launch("mce_rmsnorm");
}

// =========================================================================
// SwiGLU  (reference: csrc/kernels/swiglu.cu:8-27)
// out[t, j] = silu(g) * u, g = gate_up[t, j], u = gate_up[t, I + j].
// Grid-stride over 8-element groups of the output; every row is computed.
// =========================================================================
template <class T>
__device__ inline float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

template <class T>
__global__ __launch_bounds__(256) void swiglu_vec_kernel(
    const uint16_t *__restrict__ gu, uint16_t *__restrict__ out, int64_t rows,
    int64_t inter, int64_t in_stride, int64_t out_stride) {
  const int64_t groups_per_row = inter >> 3;
  const int64_t total = rows * groups_per_row;
  for (int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gi < total;
       gi += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = gi / groups_per_row;
    const int64_t c = (gi - r * groups_per_row) << 3;
    const uint16_t *src = gu + r * in_stride + c;
    u32x4 g = *reinterpret_cast<const u32x4 *>(src);
    u32x4 u = *reinterpret_cast<const u32x4 *>(src + inter);
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = pack2<T>(silu_mul<T>(T::lo(g[k]), T::lo(u[k])),
                      silu_mul<T>(T::hi(g[k]), T::hi(u[k])));
    *reinterpret_cast<u32x4 *>(out + r * out_stride + c) = o;
  }
}

template <class T>
__global__ __launch_bounds__(256) void swiglu_generic_kernel(
    const uint16_t *__restrict__ gu, uint16_t *__restrict__ out, int64_t rows,
    int64_t inter, int64_t in_stride, int64_t out_stride) {
  const int64_t total = rows * inter;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / inter, c = i - r * inter;
    const uint16_t *src = gu + r * in_stride + c;
    out[r * out_stride + c] =
        T::from_float(silu_mul<T>(T::lo(src[0]), T::lo(src[inter])));
  }
}

template <class T>
static int swiglu_launch(const void *gate_up, void *output, int64_t rows,
                         int64_t inter, int64_t in_stride, int64_t out_stride,
                         hipStream_t st) {
  const uint16_t *gu = (const uint16_t *)gate_up;
  uint16_t *out = (uint16_t *)output;
  const bool vec = inter % 8 == 0 && in_stride % 8 == 0 &&
                   out_stride % 8 == 0 && aligned16(gu) && aligned16(out);
  const int64_t work = vec ? rows * (inter / 8) : rows * inter;
  int64_t blocks = (work + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;  // grid-stride beyond this
  if (blocks < 1) blocks = 1;
  if (vec)
    swiglu_vec_kernel<T><<<(unsigned)blocks, 256, 0, st>>>(gu, out, rows, inter, in_stride, out_stride);
  else
    swiglu_generic_kernel<T><<<(unsigned)blocks, 256, 0, st>>>(gu, out, rows, inter, in_stride, out_stride);
  return check_launch("mce_swiglu");
}

// =========================================================================
// Paged KV store  (reference: csrc/kernels/paged_kv.cu:7-43)
// One lane per 16-byte piece of one (token, head) row; K and V both.
// Bit-exact copy.  Slots < 0 or beyond the pool are skipped.
// =========================================================================
__global__ __launch_bounds__(256) void kv_store_vec_kernel(
    const uint16_t *__restrict__ key, const uint16_t *__restrict__ value,
    uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    const int32_t *__restrict__ slots, int64_t num_tokens, int heads,
    int head_dim, int block_size, int64_t num_slots, int64_t ks_tok,
    int64_t ks_head, int64_t vs_tok, int64_t vs_head) {
  const int pieces = head_dim >> 3;
  const int64_t per_tok = (int64_t)heads * pieces;
  const int64_t total = num_tokens * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / per_tok;
    const int rem = (int)(i - n * per_tok);
    const int h = rem / pieces, p = rem - h * pieces;
    const int64_t s = slots[n];
    if (s < 0 || s >= num_slots) continue;
    // [block, offset, head] rows are contiguous in slot order.
    const int64_t dst = (s * heads + h) * head_dim + p * 8;
    *reinterpret_cast<u32x4 *>(kc + dst) =
        *reinterpret_cast<const u32x4 *>(key + n * ks_tok + h * ks_head + p * 8);
    *reinterpret_cast<u32x4 *>(vc + dst) =
        *reinterpret_cast<const u32x4 *>(value + n * vs_tok + h * vs_head + p * 8);
  }
}

// head_dim 128 with 16-byte aligned rows: one workgroup per KVS_TOK tokens.
// A pass of the 256 threads covers 16 head rows (16 threads x 16 bytes per
// 256-byte row); the workgroup's rows are (token, K or V, head) in that order.
// The source rows do not depend on the slots, so every thread issues all of
// its row and slot loads unconditionally (indices clamped into the batch; a
// per-lane condition would compile to a branch that waits for each load) and
// then stores the rows whose slot is valid: one memory round trip per thread.
// 32-bit index math throughout (the host checks the ranges).
constexpr int KVS_TOK = 4;
constexpr int KVS_MAX_PASS = 8;  // rows per thread: 2 * heads * KVS_TOK / 16

__global__ __launch_bounds__(256) void kv_store_d128_kernel(
    const uint16_t *__restrict__ key, const uint16_t *__restrict__ value,
    uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, const int32_t *__restrict__ slots,
    int num_tokens, int heads, int64_t num_slots, int64_t ks_tok, int64_t ks_head,
    int64_t vs_tok, int64_t vs_head) {
  const int p = threadIdx.x & 15, r0 = threadIdx.x >> 4;
  const int rows = 2 * heads * KVS_TOK;
  const int npass = (rows + 15) >> 4;  // uniform
  const int t0 = blockIdx.x * KVS_TOK;
  u32x4 val[KVS_MAX_PASS];
  int32_t sl[KVS_MAX_PASS];
#pragma unroll
  for (int j = 0; j < KVS_MAX_PASS; ++j) {
    if (j >= npass) break;
    const int r = min(r0 + 16 * j, rows - 1);
    const int tt = r / (2 * heads), rem = r - tt * 2 * heads;
    const int t = min(t0 + tt, num_tokens - 1);
    const bool is_v = rem >= heads;
    const int h = is_v ? rem - heads : rem;
    const uint16_t *src = is_v ? value + t * vs_tok + h * vs_head : key + t * ks_tok + h * ks_head;
    val[j] = *reinterpret_cast<const u32x4 *>(src + 8 * p);
    sl[j] = slots[t];
  }
#pragma unroll
  for (int j = 0; j < KVS_MAX_PASS; ++j) {
    if (j >= npass) break;
    const int r = r0 + 16 * j;
    const int tt = r / (2 * heads), rem = r - tt * 2 * heads;
    const bool is_v = rem >= heads;
    const int h = is_v ? rem - heads : rem;
    const int64_t s = sl[j];
    if (r < rows && t0 + tt < num_tokens && s >= 0 && s < num_slots)
      *reinterpret_cast<u32x4 *>((is_v ? vc : kc) + (s * heads + h) * 128 + 8 * p) = val[j];
  }
}

__global__ __launch_bounds__(256) void kv_store_generic_kernel(
    const uint16_t *__restrict__ key, const uint16_t *__restrict__ value,
    uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    const int32_t *__restrict__ slots, int64_t num_tokens, int heads,
    int head_dim, int block_size, int64_t num_slots, int64_t ks_tok,
    int64_t ks_head, int64_t vs_tok, int64_t vs_head) {
  const int64_t per_tok = (int64_t)heads * head_dim;
  const int64_t total = num_tokens * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / per_tok;
    const int rem = (int)(i - n * per_tok);
    const int h = rem / head_dim, d = rem - h * head_dim;
    const int64_t s = slots[n];
    if (s < 0 || s >= num_slots) continue;
    const int64_t dst = (s * heads + h) * head_dim + d;
    kc[dst] = key[n * ks_tok + h * ks_head + d];
    vc[dst] = value[n * vs_tok + h * vs_head + d];
  }
}

// =========================================================================
// In-place RoPE  (reference: csrc/kernels/rope.cu:6-62; tables
// engine/models/llama.py:47-57)
// One lane per 4 rotation pairs of one (token, head): 8-byte loads of
// x[i..i+3] and x[i+D/2..], 16-byte loads of cos/sin.  Q heads and K heads
// share the launch (heads >= num_heads index K).
// =========================================================================
template <class T>
__device__ inline void rope_rotate4(const uint16_t *p, int half, const float *c4,
                                    const float *s4, uint16_t *out) {
  u32x2 a = *reinterpret_cast<const u32x2 *>(p);
  u32x2 b = *reinterpret_cast<const u32x2 *>(p + half);
  float x0[4] = {T::lo(a[0]), T::hi(a[0]), T::lo(a[1]), T::hi(a[1])};
  float x1[4] = {T::lo(b[0]), T::hi(b[0]), T::lo(b[1]), T::hi(b[1])};
  float r0[4], r1[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) rope_pair(x0[k], x1[k], c4[k], s4[k], r0[k], r1[k]);
  u32x2 oa, ob;
  oa[0] = pack2<T>(r0[0], r0[1]);
  oa[1] = pack2<T>(r0[2], r0[3]);
  ob[0] = pack2<T>(r1[0], r1[1]);
  ob[1] = pack2<T>(r1[2], r1[3]);
  *reinterpret_cast<u32x2 *>(out) = oa;
  *reinterpret_cast<u32x2 *>(out + half) = ob;
}

template <class T>
__global__ __launch_bounds__(256) void rope_vec_kernel(
    uint16_t *__restrict__ q, uint16_t *__restrict__ k,
    const float *__restrict__ cos_t, const float *__restrict__ sin_t,
    const int32_t *__restrict__ pos, int64_t tokens, int seq_len,
    int num_heads, int num_kv_heads, int head_dim, int64_t table_rows,
    int64_t qsb, int64_t qss, int64_t qsh, int64_t ksb, int64_t kss,
    int64_t ksh) {
  const int half = head_dim >> 1;
  const int quads = half >> 2;
  const int heads = num_heads + num_kv_heads;
  const int64_t per_tok = (int64_t)heads * quads;
  const int64_t total = tokens * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_tok;
    const int rem = (int)(i - t * per_tok);
    const int h = rem / quads, qd = rem - h * quads;
    const int64_t ps = pos[t];
    if (ps < 0 || ps >= table_rows) continue;
    const int64_t b = t / seq_len, s = t - b * seq_len;
    uint16_t *p = h < num_heads
                      ? q + b * qsb + s * qss + h * qsh
                      : k + b * ksb + s * kss + (h - num_heads) * ksh;
    floatx4 c = *reinterpret_cast<const floatx4 *>(cos_t + ps * half + qd * 4);
    floatx4 sn = *reinterpret_cast<const floatx4 *>(sin_t + ps * half + qd * 4);
    float c4[4] = {c[0], c[1], c[2], c[3]};
    float s4[4] = {sn[0], sn[1], sn[2], sn[3]};
    rope_rotate4<T>(p + qd * 4, half, c4, s4, p + qd * 4);
  }
}

// head_dim 128 with 16-byte aligned rows: a head row is rotated by 8 lanes,
// lane l8 taking pairs 8 l8 .. 8 l8 + 7 (one 16-byte load from each half of
// the row, two 16-byte loads of cos and of sin).  Same rope_pair arithmetic
// as the kernels above, so the results are bit-identical to them.
template <class T>
__device__ inline void rope_rotate8(const uint16_t *p, const float *cr, const float *sr, int l8,
                                    u32x4 &oa, u32x4 &ob) {
  const u32x4 a = *reinterpret_cast<const u32x4 *>(p + 8 * l8);
  const u32x4 b = *reinterpret_cast<const u32x4 *>(p + 64 + 8 * l8);
  const floatx4 c0 = *reinterpret_cast<const floatx4 *>(cr + 8 * l8);
  const floatx4 c1 = *reinterpret_cast<const floatx4 *>(cr + 8 * l8 + 4);
  const floatx4 s0 = *reinterpret_cast<const floatx4 *>(sr + 8 * l8);
  const floatx4 s1 = *reinterpret_cast<const floatx4 *>(sr + 8 * l8 + 4);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float c_lo = k < 2 ? c0[2 * k] : c1[2 * k - 4], c_hi = k < 2 ? c0[2 * k + 1] : c1[2 * k - 3];
    const float s_lo = k < 2 ? s0[2 * k] : s1[2 * k - 4], s_hi = k < 2 ? s0[2 * k + 1] : s1[2 * k - 3];
    float r0a, r1a, r0b, r1b;
    rope_pair(T::lo(a[k]), T::lo(b[k]), c_lo, s_lo, r0a, r1a);
    rope_pair(T::hi(a[k]), T::hi(b[k]), c_hi, s_hi, r0b, r1b);
    oa[k] = pack2<T>(r0a, r0b);
    ob[k] = pack2<T>(r1a, r1b);
  }
}

// the two 16-byte halves of lane l8's piece of a 128-wide row
__device__ inline void store_row8(uint16_t *dst, int l8, const u32x4 &lo, const u32x4 &hi) {
  *reinterpret_cast<u32x4 *>(dst + 8 * l8) = lo;
  *reinterpret_cast<u32x4 *>(dst + 64 + 8 * l8) = hi;
}

// rope_inplace for head_dim 128: one workgroup per ROPE_TOK tokens, a pass of
// 256 threads covering 32 head rows (query heads, then key heads, per token).
constexpr int ROPE_TOK = 2;

template <class T>
__global__ __launch_bounds__(256) void rope_d128_kernel(
    uint16_t *__restrict__ q, uint16_t *__restrict__ k, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int32_t *__restrict__ pos, int tokens, int seq_len,
    int num_heads, int num_kv_heads, int64_t table_rows, int64_t qsb, int64_t qss, int64_t qsh,
    int64_t ksb, int64_t kss, int64_t ksh) {
  const int l8 = threadIdx.x & 7;
  const int heads = num_heads + num_kv_heads;
  const int rows = heads * ROPE_TOK;
  const int t0 = blockIdx.x * ROPE_TOK;
  for (int r = threadIdx.x >> 3; r < rows; r += 32) {
    const int tt = r / heads, h = r - tt * heads;
    const int t = t0 + tt;
    if (t >= tokens) break;
    const int64_t ps = pos[t];
    if (ps < 0 || ps >= table_rows) continue;
    const int b = t / seq_len, s = t - b * seq_len;
    uint16_t *p = h < num_heads ? q + b * qsb + s * qss + h * qsh
                                : k + b * ksb + s * kss + (h - num_heads) * ksh;
    u32x4 lo, hi;
    rope_rotate8<T>(p, cos_t + ps * 64, sin_t + ps * 64, l8, lo, hi);
    store_row8(p, l8, lo, hi);
  }
}

// rope_kv_store for head_dim 128: like rope_d128_kernel over the rows
// (query heads, key heads, value heads) of each token.
template <class T>
__global__ __launch_bounds__(256) void rope_kv_store_d128_kernel(
    uint16_t *__restrict__ q, uint16_t *__restrict__ q_out, uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    const float *__restrict__ cos_t, const float *__restrict__ sin_t,
    const int32_t *__restrict__ pos, const int32_t *__restrict__ slots, int tokens,
    int num_heads, int num_kv_heads, int64_t table_rows, int64_t num_slots, int64_t qst,
    int64_t qsh, int64_t kst, int64_t ksh, int64_t vst, int64_t vsh) {
  const int l8 = threadIdx.x & 7;
  const int heads = num_heads + 2 * num_kv_heads;
  const int rows = heads * ROPE_TOK;
  const int t0 = blockIdx.x * ROPE_TOK;
  for (int r = threadIdx.x >> 3; r < rows; r += 32) {
    const int tt = r / heads, h = r - tt * heads;
    const int t = t0 + tt;
    if (t >= tokens) break;
    const int64_t ps = pos[t];
    const bool in_table = ps >= 0 && ps < table_rows;
    const float *cr = cos_t + (in_table ? ps : 0) * 64, *sr = sin_t + (in_table ? ps : 0) * 64;
    if (h < num_heads) {
      uint16_t *p = q + t * qst + h * qsh;
      uint16_t *dst = q_out ? q_out + ((int64_t)t * num_heads + h) * 128 : p;
      if (in_table) {
        u32x4 lo, hi;
        rope_rotate8<T>(p, cr, sr, l8, lo, hi);
        store_row8(dst, l8, lo, hi);
      } else if (q_out) {
        store_row8(dst, l8, *reinterpret_cast<const u32x4 *>(p + 8 * l8),
                   *reinterpret_cast<const u32x4 *>(p + 64 + 8 * l8));
      }
      continue;
    }
    const int64_t sl = slots[t];
    const bool store = sl >= 0 && sl < num_slots;
    if (h < num_heads + num_kv_heads) {
      const int hk = h - num_heads;
      uint16_t *p = k + t * kst + hk * ksh;
      u32x4 lo, hi;
      if (in_table) {
        rope_rotate8<T>(p, cr, sr, l8, lo, hi);
        store_row8(p, l8, lo, hi);
      } else {
        lo = *reinterpret_cast<const u32x4 *>(p + 8 * l8);
        hi = *reinterpret_cast<const u32x4 *>(p + 64 + 8 * l8);
      }
      if (store) store_row8(kc + (sl * num_kv_heads + hk) * 128, l8, lo, hi);
    } else if (store) {
      const int hv = h - num_heads - num_kv_heads;
      const uint16_t *p = v + t * vst + hv * vsh;
      store_row8(vc + (sl * num_kv_heads + hv) * 128, l8,
                 *reinterpret_cast<const u32x4 *>(p + 8 * l8),
                 *reinterpret_cast<const u32x4 *>(p + 64 + 8 * l8));
    }
  }
}

// RoPE of q and k in place plus the paged store of the rotated k and of v,
// in one launch (the engine applies rope_inplace and paged_kv_store back to
// back on the same tokens).  One lane per 4 rotation pairs of one (token,
// head): head slots [0, Hq) are query heads (rotated in place, or into the
// contiguous [N, Hq, D] rows of q_out when given), [Hq, Hq + Hkv) key heads
// (rotated in place, then written to key_cache[slot]), [Hq + Hkv, Hq + 2 Hkv)
// value heads (copied to value_cache[slot]).  Same arithmetic as
// rope_vec_kernel, so the results are bit-identical to the two separate ops;
// positions outside the table leave q/k unrotated and slots outside the pool
// are skipped, as in the separate ops.
template <class T>
__global__ __launch_bounds__(256) void rope_kv_store_vec_kernel(
    uint16_t *__restrict__ q, uint16_t *__restrict__ q_out, uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
    const float *__restrict__ cos_t, const float *__restrict__ sin_t,
    const int32_t *__restrict__ pos, const int32_t *__restrict__ slots, int64_t tokens,
    int num_heads, int num_kv_heads, int head_dim, int64_t table_rows, int64_t num_slots,
    int64_t qst, int64_t qsh, int64_t kst, int64_t ksh, int64_t vst, int64_t vsh) {
  const int half = head_dim >> 1;
  const int quads = half >> 2;
  const int heads = num_heads + 2 * num_kv_heads;
  const int64_t per_tok = (int64_t)heads * quads;
  const int64_t total = tokens * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_tok;
    const int rem = (int)(i - t * per_tok);
    const int h = rem / quads, qd = rem - h * quads;
    const int64_t ps = pos[t];
    const bool in_table = ps >= 0 && ps < table_rows;
    if (h < num_heads) {
      const uint16_t *p = q + t * qst + h * qsh + qd * 4;
      uint16_t *dst = q_out ? q_out + (t * num_heads + h) * head_dim + qd * 4
                            : q + t * qst + h * qsh + qd * 4;
      if (in_table) {
        floatx4 c = *reinterpret_cast<const floatx4 *>(cos_t + ps * half + qd * 4);
        floatx4 sn = *reinterpret_cast<const floatx4 *>(sin_t + ps * half + qd * 4);
        float c4[4] = {c[0], c[1], c[2], c[3]};
        float s4[4] = {sn[0], sn[1], sn[2], sn[3]};
        rope_rotate4<T>(p, half, c4, s4, dst);
      } else if (q_out) {
        *reinterpret_cast<u32x2 *>(dst) = *reinterpret_cast<const u32x2 *>(p);
        *reinterpret_cast<u32x2 *>(dst + half) = *reinterpret_cast<const u32x2 *>(p + half);
      }
      continue;
    }
    const int64_t sl = slots[t];
    const bool store = sl >= 0 && sl < num_slots;
    if (h < num_heads + num_kv_heads) {
      const int hk = h - num_heads;
      uint16_t *p = k + t * kst + hk * ksh + qd * 4;
      if (in_table) {
        floatx4 c = *reinterpret_cast<const floatx4 *>(cos_t + ps * half + qd * 4);
        floatx4 sn = *reinterpret_cast<const floatx4 *>(sin_t + ps * half + qd * 4);
        float c4[4] = {c[0], c[1], c[2], c[3]};
        float s4[4] = {sn[0], sn[1], sn[2], sn[3]};
        rope_rotate4<T>(p, half, c4, s4, p);
      }
      if (store) {
        uint16_t *dst = kc + (sl * num_kv_heads + hk) * head_dim + qd * 4;
        *reinterpret_cast<u32x2 *>(dst) = *reinterpret_cast<const u32x2 *>(p);
        *reinterpret_cast<u32x2 *>(dst + half) = *reinterpret_cast<const u32x2 *>(p + half);
      }
    } else if (store) {
      const int hv = h - num_heads - num_kv_heads;
      const uint16_t *p = v + t * vst + hv * vsh + qd * 4;
      uint16_t *dst = vc + (sl * num_kv_heads + hv) * head_dim + qd * 4;
      *reinterpret_cast<u32x2 *>(dst) = *reinterpret_cast<const u32x2 *>(p);
      *reinterpret_cast<u32x2 *>(dst + half) = *reinterpret_cast<const u32x2 *>(p + half);
    }
  }
}

template <class T>
__global__ __launch_bounds__(256) void rope_generic_kernel(
    uint16_t *__restrict__ q, uint16_t *__restrict__ k,
    const float *__restrict__ cos_t, const float *__restrict__ sin_t,
    const int32_t *__restrict__ pos, int64_t tokens, int seq_len,
    int num_heads, int num_kv_heads, int head_dim, int64_t table_rows,
    int64_t qsb, int64_t qss, int64_t qsh, int64_t ksb, int64_t kss,
    int64_t ksh) {
  const int half = head_dim >> 1;
  const int heads = num_heads + num_kv_heads;
  const int64_t per_tok = (int64_t)heads * half;
  const int64_t total = tokens * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_tok;
    const int rem = (int)(i - t * per_tok);
    const int h = rem / half, d = rem - h * half;
    const int64_t ps = pos[t];
    if (ps < 0 || ps >= table_rows) continue;
    const int64_t b = t / seq_len, s = t - b * seq_len;
    uint16_t *p = h < num_heads
                      ? q + b * qsb + s * qss + h * qsh
                      : k + b * ksb + s * kss + (h - num_heads) * ksh;
    const float c = cos_t[ps * half + d], sn = sin_t[ps * half + d];
    const float x0 = T::lo(p[d]), x1 = T::lo(p[d + half]);
    p[d] = T::from_float(x0 * c - x1 * sn);
    p[d + half] = T::from_float(x0 * sn + x1 * c);
  }
}

static unsigned grid_for(int64_t work) {
  int64_t blocks = (work + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;
  return (unsigned)(blocks < 1 ? 1 : blocks);
}

}  // namespace mce

using namespace mce;

extern "C" int mce_rmsnorm(int dtype, const void *input, const void *weight,
                           void *output, int64_t rows, int64_t hidden,
                           int64_t in_row_stride, int64_t out_row_stride,
                           float eps, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "mce_rmsnorm: unknown dtype %d", dtype);
  MCE_REQUIRE(rows >= 0 && hidden >= 1 && hidden <= (1 << 24),
              "mce_rmsnorm: bad shape rows=%lld hidden=%lld", (long long)rows, (long long)hidden);
  MCE_REQUIRE(in_row_stride >= hidden && out_row_stride >= hidden,
              "mce_rmsnorm: row stride smaller than hidden size");
  if (rows == 0) return MCE_OK;
  MCE_REQUIRE(input && weight && output, "mce_rmsnorm: null pointer");
  MCE_REQUIRE(rows < ((int64_t)1 << 31) - 1, "mce_rmsnorm: too many rows");
  hipStream_t st = (hipStream_t)stream;
  return dtype == MCE_F16
             ? rmsnorm_launch<F16T>(input, weight, output, rows, hidden, in_row_stride, out_row_stride, eps, st)
             : rmsnorm_launch<BF16T>(input, weight, output, rows, hidden, in_row_stride, out_row_stride, eps, st);
}

extern "C" int mce_swiglu(int dtype, const void *gate_up, void *output,
                          int64_t rows, int64_t inter, int64_t in_row_stride,
                          int64_t out_row_stride, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "mce_swiglu: unknown dtype %d", dtype);
  MCE_REQUIRE(rows >= 0 && inter >= 0, "mce_swiglu: bad shape");
  MCE_REQUIRE(in_row_stride >= 2 * inter && out_row_stride >= inter,
              "mce_swiglu: row stride smaller than row");
  if (rows == 0 || inter == 0) return MCE_OK;
  MCE_REQUIRE(gate_up && output, "mce_swiglu: null pointer");
  hipStream_t st = (hipStream_t)stream;
  return dtype == MCE_F16
             ? swiglu_launch<F16T>(gate_up, output, rows, inter, in_row_stride, out_row_stride, st)
             : swiglu_launch<BF16T>(gate_up, output, rows, inter, in_row_stride, out_row_stride, st);
}

extern "C" int mce_paged_kv_store(int dtype, const void *key, const void *value,
                                  void *key_cache, void *value_cache,
                                  const int32_t *slot_mapping,
                                  int64_t num_tokens, int num_kv_heads,
                                  int head_dim, int block_size,
                                  int64_t num_blocks, int64_t key_stride_tok,
                                  int64_t key_stride_head,
                                  int64_t value_stride_tok,
                                  int64_t value_stride_head, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "mce_paged_kv_store: unknown dtype %d", dtype);
  MCE_REQUIRE(num_tokens >= 0 && num_kv_heads >= 1 && head_dim >= 1 &&
                  block_size >= 1 && num_blocks >= 0,
              "mce_paged_kv_store: bad shape");
  if (num_tokens == 0 || num_blocks == 0) return MCE_OK;
  MCE_REQUIRE(key && value && key_cache && value_cache && slot_mapping,
              "mce_paged_kv_store: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t num_slots = num_blocks * block_size;
  const bool vec = head_dim % 8 == 0 && key_stride_tok % 8 == 0 &&
                   key_stride_head % 8 == 0 && value_stride_tok % 8 == 0 &&
                   value_stride_head % 8 == 0 && aligned16(key) &&
                   aligned16(value) && aligned16(key_cache) &&
                   aligned16(value_cache);
  const int64_t work = num_tokens * num_kv_heads * (vec ? head_dim / 8 : head_dim);
  if (vec && head_dim == 128 && 2 * num_kv_heads * KVS_TOK <= 16 * KVS_MAX_PASS &&
      num_tokens < ((int64_t)1 << 31) - KVS_TOK)
    kv_store_d128_kernel<<<(unsigned)((num_tokens + KVS_TOK - 1) / KVS_TOK), 256, 0, st>>>(
        (const uint16_t *)key, (const uint16_t *)value, (uint16_t *)key_cache,
        (uint16_t *)value_cache, slot_mapping, (int)num_tokens, num_kv_heads, num_slots,
        key_stride_tok, key_stride_head, value_stride_tok, value_stride_head);
  else if (vec)
    kv_store_vec_kernel<<<grid_for(work), 256, 0, st>>>(
        (const uint16_t *)key, (const uint16_t *)value, (uint16_t *)key_cache,
        (uint16_t *)value_cache, slot_mapping, num_tokens, num_kv_heads,
        head_dim, block_size, num_slots, key_stride_tok, key_stride_head,
        value_stride_tok, value_stride_head);
  else
    kv_store_generic_kernel<<<grid_for(work), 256, 0, st>>>(
        (const uint16_t *)key, (const uint16_t *)value, (uint16_t *)key_cache,
        (uint16_t *)value_cache, slot_mapping, num_tokens, num_kv_heads,
        head_dim, block_size, num_slots, key_stride_tok, key_stride_head,
        value_stride_tok, value_stride_head);
  return check_launch("mce_paged_kv_store");
}

extern "C" int mce_rope_inplace(int dtype, void *query, void *key,
                                const float *cos_table, const float *sin_table,
                                const int32_t *positions, int batch,
                                int seq_len, int num_heads, int num_kv_heads,
                                int head_dim, int64_t table_rows,
                                int64_t q_stride_b, int64_t q_stride_s,
                                int64_t q_stride_h, int64_t k_stride_b,
                                int64_t k_stride_s, int64_t k_stride_h,
                                void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "mce_rope_inplace: unknown dtype %d", dtype);
  MCE_REQUIRE(batch >= 0 && seq_len >= 0 && num_heads >= 0 && head_dim >= 2 &&
                  head_dim % 2 == 0 && table_rows >= 0,
              "mce_rope_inplace: bad shape");
  if (!key) num_kv_heads = 0;
  MCE_REQUIRE(num_kv_heads >= 0, "mce_rope_inplace: bad num_kv_heads");
  const int64_t tokens = (int64_t)batch * seq_len;
  if (tokens == 0 || num_heads + num_kv_heads == 0) return MCE_OK;
  MCE_REQUIRE(query && cos_table && sin_table && positions,
              "mce_rope_inplace: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int half = head_dim / 2;
  bool vec = half % 4 == 0 && q_stride_b % 4 == 0 && q_stride_s % 4 == 0 &&
             q_stride_h % 4 == 0 && (reinterpret_cast<uintptr_t>(query) & 7) == 0 &&
             aligned16(cos_table) && aligned16(sin_table);
  if (key)
    vec = vec && k_stride_b % 4 == 0 && k_stride_s % 4 == 0 &&
          k_stride_h % 4 == 0 && (reinterpret_cast<uintptr_t>(key) & 7) == 0;
  const int heads = num_heads + num_kv_heads;
  uint16_t *q = (uint16_t *)query, *k = (uint16_t *)key;
  const bool d128 = head_dim == 128 && tokens < ((int64_t)1 << 31) - ROPE_TOK &&
                    q_stride_b % 8 == 0 && q_stride_s % 8 == 0 && q_stride_h % 8 == 0 &&
                    aligned16(query) && aligned16(cos_table) && aligned16(sin_table) &&
                    (!key || (k_stride_b % 8 == 0 && k_stride_s % 8 == 0 &&
                              k_stride_h % 8 == 0 && aligned16(key)));
  if (d128) {
    const unsigned grid = (unsigned)((tokens + ROPE_TOK - 1) / ROPE_TOK);
    if (dtype == MCE_F16)
      rope_d128_kernel<F16T><<<grid, 256, 0, st>>>(q, k, cos_table, sin_table, positions,
                                                   (int)tokens, seq_len, num_heads, num_kv_heads,
                                                   table_rows, q_stride_b, q_stride_s, q_stride_h,
                                                   k_stride_b, k_stride_s, k_stride_h);
    else
      rope_d128_kernel<BF16T><<<grid, 256, 0, st>>>(q, k, cos_table, sin_table, positions,
                                                    (int)tokens, seq_len, num_heads, num_kv_heads,
                                                    table_rows, q_stride_b, q_stride_s, q_stride_h,
                                                    k_stride_b, k_stride_s, k_stride_h);
  } else if (vec) {
    const int64_t work = tokens * heads * (half / 4);
    if (dtype == MCE_F16)
      rope_vec_kernel<F16T><<<grid_for(work), 256, 0, st>>>(q, k, cos_table, sin_table, positions, tokens, seq_len, num_heads, num_kv_heads, head_dim, table_rows, q_stride_b, q_stride_s, q_stride_h, k_stride_b, k_stride_s, k_stride_h);
    else
      rope_vec_kernel<BF16T><<<grid_for(work), 256, 0, st>>>(q, k, cos_table, sin_table, positions, tokens, seq_len, num_heads, num_kv_heads, head_dim, table_rows, q_stride_b, q_stride_s, q_stride_h, k_stride_b, k_stride_s, k_stride_h);
  } else {
    const int64_t work = tokens * heads * half;
    if (dtype == MCE_F16)
      rope_generic_kernel<F16T><<<grid_for(work), 256, 0, st>>>(q, k, cos_table, sin_table, positions, tokens, seq_len, num_heads, num_kv_heads, head_dim, table_rows, q_stride_b, q_stride_s, q_stride_h, k_stride_b, k_stride_s, k_stride_h);
    else
      rope_generic_kernel<BF16T><<<grid_for(work), 256, 0, st>>>(q, k, cos_table, sin_table, positions, tokens, seq_len, num_heads, num_kv_heads, head_dim, table_rows, q_stride_b, q_stride_s, q_stride_h, k_stride_b, k_stride_s, k_stride_h);
  }
  return check_launch("mce_rope_inplace");
}

extern "C" int mce_rope_kv_store(int dtype, void *query, void *query_out, void *key,
                                 const void *value,
                                 void *key_cache, void *value_cache,
                                 const float *cos_table, const float *sin_table,
                                 const int32_t *positions, const int32_t *slot_mapping,
                                 int64_t num_tokens, int num_heads, int num_kv_heads,
                                 int head_dim, int64_t table_rows, int block_size,
                                 int64_t num_blocks, int64_t q_stride_tok,
                                 int64_t q_stride_head, int64_t k_stride_tok,
                                 int64_t k_stride_head, int64_t v_stride_tok,
                                 int64_t v_stride_head, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "mce_rope_kv_store: unknown dtype %d", dtype);
  MCE_REQUIRE(num_tokens >= 0 && num_heads >= 0 && num_kv_heads >= 1 && head_dim >= 2 &&
                  head_dim % 2 == 0 && table_rows >= 0 && block_size >= 1 && num_blocks >= 0,
              "mce_rope_kv_store: bad shape");
  if (num_tokens == 0) return MCE_OK;
  MCE_REQUIRE(query && key && value && key_cache && value_cache && cos_table && sin_table &&
                  positions && slot_mapping,
              "mce_rope_kv_store: null pointer");
  const int half = head_dim / 2;
  const bool vec = half % 4 == 0 && q_stride_tok % 4 == 0 && q_stride_head % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(query_out) & 7) == 0 &&
                   k_stride_tok % 4 == 0 && k_stride_head % 4 == 0 && v_stride_tok % 4 == 0 &&
                   v_stride_head % 4 == 0 && ((reinterpret_cast<uintptr_t>(query) |
                                               reinterpret_cast<uintptr_t>(key) |
                                               reinterpret_cast<uintptr_t>(value) |
                                               reinterpret_cast<uintptr_t>(key_cache) |
                                               reinterpret_cast<uintptr_t>(value_cache)) &
                                              7) == 0 &&
                   aligned16(cos_table) && aligned16(sin_table);
  if (!vec) {
    // any layout: the two separate ops (query rows copied out first)
    if (query_out) {
      const size_t row = (size_t)head_dim * 2;
      for (int h = 0; h < num_heads; ++h)
        if (hipMemcpy2DAsync((char *)query_out + h * row, (size_t)num_heads * row,
                             (const char *)query + h * q_stride_head * 2,
                             (size_t)q_stride_tok * 2, row, (size_t)num_tokens,
                             hipMemcpyDeviceToDevice, (hipStream_t)stream) != hipSuccess)
          return set_error(MCE_ERR_LAUNCH, "mce_rope_kv_store: query copy failed");
      query = query_out;
      q_stride_tok = (int64_t)num_heads * head_dim;
      q_stride_head = head_dim;
    }
    int rc = mce_rope_inplace(dtype, query, key, cos_table, sin_table, positions,
                              (int)num_tokens, 1, num_heads, num_kv_heads, head_dim, table_rows,
                              q_stride_tok, 0, q_stride_head, k_stride_tok, 0, k_stride_head,
                              stream);
    if (rc != MCE_OK) return rc;
    return mce_paged_kv_store(dtype, key, value, key_cache, value_cache, slot_mapping,
                              num_tokens, num_kv_heads, head_dim, block_size, num_blocks,
                              k_stride_tok, k_stride_head, v_stride_tok, v_stride_head, stream);
  }
  MCE_REQUIRE(num_tokens < ((int64_t)1 << 31) - ROPE_TOK, "mce_rope_kv_store: too many tokens");
  hipStream_t st = (hipStream_t)stream;
  const int64_t num_slots = num_blocks * block_size;
  const bool d128 = head_dim == 128 && q_stride_tok % 8 == 0 && q_stride_head % 8 == 0 &&
                    k_stride_tok % 8 == 0 && k_stride_head % 8 == 0 && v_stride_tok % 8 == 0 &&
                    v_stride_head % 8 == 0 && aligned16(query) && aligned16(key) &&
                    aligned16(value) && aligned16(key_cache) && aligned16(value_cache) &&
                    (!query_out || aligned16(query_out));
  if (d128) {
    const unsigned grid = (unsigned)((num_tokens + ROPE_TOK - 1) / ROPE_TOK);
#define MCE_RKV128(TT)                                                                           \
  rope_kv_store_d128_kernel<TT><<<grid, 256, 0, st>>>(                                           \
      (uint16_t *)query, (uint16_t *)query_out, (uint16_t *)key, (const uint16_t *)value,        \
      (uint16_t *)key_cache, (uint16_t *)value_cache, cos_table, sin_table, positions,           \
      slot_mapping, (int)num_tokens, num_heads, num_kv_heads, table_rows, num_slots,             \
      q_stride_tok, q_stride_head, k_stride_tok, k_stride_head, v_stride_tok, v_stride_head)
    if (dtype == MCE_F16)
      MCE_RKV128(F16T);
    else
      MCE_RKV128(BF16T);
#undef MCE_RKV128
    return check_launch("mce_rope_kv_store");
  }
  const int64_t work = num_tokens * (num_heads + 2 * num_kv_heads) * (half / 4);
#define MCE_RKV(TT)                                                                              \
  rope_kv_store_vec_kernel<TT><<<grid_for(work), 256, 0, st>>>(                                  \
      (uint16_t *)query, (uint16_t *)query_out, (uint16_t *)key, (const uint16_t *)value,        \
      (uint16_t *)key_cache,                                                                     \
      (uint16_t *)value_cache, cos_table, sin_table, positions, slot_mapping, num_tokens,        \
      num_heads, num_kv_heads, head_dim, table_rows, num_slots, q_stride_tok, q_stride_head,     \
      k_stride_tok, k_stride_head, v_stride_tok, v_stride_head)
  if (dtype == MCE_F16)
    MCE_RKV(F16T);
  else
    MCE_RKV(BF16T);
#undef MCE_RKV
  return check_launch("mce_rope_kv_store");
}
