// Device-side preparation of the next decode step, so that a captured decode
// graph can be replayed step after step with no host work in between:
//   * mce_argmax_rows: greedy token of each logits row (the reference's
//     benchmark loop takes torch.argmax of the logits between replays,
//     benchmarks/benchmark_engine.py:255-265);
//   * mce_decode_advance: appends those tokens to a token log, moves every
//     sequence one position on and recomputes its slot from the device block
//     table (the reference computes positions, context lengths and slots on
//     the host and copies them in before every replay, engine/runner.py:
//     39-60,153-176, with the slot rule of engine/cache.py:48-57).
// Both are index work: bit-exact against the allocator's slot rule and
// torch.argmax.
#include "mce_common.h"

namespace mce {

constexpr int AM_THREADS = 512;

// (value, index) order of argmax: larger value first, NaN above every number
// (as torch.argmax ranks it), the lower index among equals.
__device__ inline bool am_better(float a, int64_t ia, float b, int64_t ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

// Order key of argmax's value rule as an unsigned integer: larger keys are
// larger values, NaN (any sign or payload) above +inf, -0 equal to +0 (equal
// values are then ranked by index alone, as torch.argmax does).
__device__ inline uint32_t am_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  // negative: ~u; positive: u with the top bit set (selects, no branches)
  uint32_t k = u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
  k = (u << 1) == 0 ? 0x80000000u : k;  // +0 and -0
  return v != v ? 0xffffffffu : k;
}

// (key, index) order: larger key first, the lower index among equals.
__device__ inline bool am_key_better(uint32_t ka, int ia, uint32_t kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// Rows split over AMP_PARTS workgroups each (16-byte aligned rows): every
// workgroup scans its slice of the row with 16-byte loads and writes its best
// (key, column) as one 64-bit value, key << 32 | ~column, whose unsigned order
// is argmax's order (a larger key first, then the lower column); a second
// kernel takes the maximum of each row's parts.  Spreading a row over many CUs
// matters: the scan costs ~14 VALU instructions per element, which on the 8
// CUs of one workgroup per row would take ~14 us for an 8 x 128256 batch.
constexpr int AMP_THREADS = 256;
constexpr int AMP_CHUNKS = 4;            // 16-byte chunks per thread per pass
constexpr int AMP_COLS_PER_PART = 4096;  // columns per workgroup (at most AMP_MAX_PARTS parts)
constexpr int AMP_MAX_PARTS = 64;

__host__ __device__ inline int argmax_parts(int64_t cols) {
  const int64_t p = (cols + AMP_COLS_PER_PART - 1) / AMP_COLS_PER_PART;
  return (int)(p < 1 ? 1 : (p > AMP_MAX_PARTS ? AMP_MAX_PARTS : p));
}

__device__ inline uint64_t am_pack(uint32_t key, int col) {
  return ((uint64_t)key << 32) | (uint32_t)~(uint32_t)col;
}

template <class T>
__global__ __launch_bounds__(AMP_THREADS) void argmax_part_kernel(
    const uint16_t *__restrict__ x, int cols, int64_t stride, int parts,
    uint64_t *__restrict__ part_out) {
  const int p = blockIdx.x, row = blockIdx.y;
  const uint16_t *xr = x + (int64_t)row * stride;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n8 = cols >> 3;
  const int span = (n8 + parts - 1) / parts;  // 8-value chunks per part
  const int lo = p * span, hi = min(n8, lo + span);
  uint32_t bk = 0;  // below every value's key
  int bi = cols;    // past the end: loses to every real element
  for (int base = lo; base < hi; base += AMP_THREADS * AMP_CHUNKS) {
    // unconditional loads (past the slice: its last chunk again, keys masked),
    // so each chunk's scan waits for that load only
    u32x4 v[AMP_CHUNKS];
#pragma unroll
    for (int k = 0; k < AMP_CHUNKS; ++k) {
      const int c8 = base + k * AMP_THREADS + tid;
      v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(xr) +
                                        (c8 < hi ? c8 : hi - 1));
    }
    // branch-free scan in increasing column order (strict > keeps the first
    // of equal keys); chunks past the slice get key 0, which never wins
#pragma unroll
    for (int k = 0; k < AMP_CHUNKS; ++k) {
      const int c8 = base + k * AMP_THREADS + tid;
      const uint32_t in_row = c8 < hi ? 0xffffffffu : 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t k0 = am_key(T::lo(v[k][e])) & in_row;
        const uint32_t k1 = am_key(T::hi(v[k][e])) & in_row;
        const bool t0 = k0 > bk;
        bk = t0 ? k0 : bk;
        bi = t0 ? c8 * 8 + 2 * e : bi;
        const bool t1 = k1 > bk;
        bk = t1 ? k1 : bk;
        bi = t1 ? c8 * 8 + 2 * e + 1 : bi;
      }
    }
  }
  if (p == parts - 1) {  // columns past the last whole 8-value chunk
    const int c = n8 * 8 + tid;
    if (c < cols) {
      const uint32_t kc = am_key(T::lo(xr[c]));
      if (am_key_better(kc, c, bk, bi)) {
        bk = kc;
        bi = c;
      }
    }
  }
  // the order is total, so the reduction order does not change the result
  uint64_t best = bi < cols ? am_pack(bk, bi) : 0;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const uint64_t o = __shfl_xor(best, d, 64);
    best = o > best ? o : best;
  }
  __shared__ uint64_t wbest[AMP_THREADS / 64];
  if (lane == 0) wbest[w] = best;
  __syncthreads();
  if (tid == 0) {
    for (int k = 1; k < AMP_THREADS / 64; ++k) best = wbest[k] > best ? wbest[k] : best;
    part_out[(int64_t)row * parts + p] = best;
  }
}

// one wave per row: the maximum of the row's part values; the column is the
// complement of its low 32 bits (a row of only empty parts -- not possible for
// cols >= 1 -- would give column 0)
__global__ __launch_bounds__(64) void argmax_final_kernel(const uint64_t *__restrict__ part,
                                                          int parts,
                                                          int64_t *__restrict__ out) {
  const int row = blockIdx.x, lane = threadIdx.x;
  uint64_t best = 0;
  for (int k = lane; k < parts; k += 64) {
    const uint64_t v = part[(int64_t)row * parts + k];
    best = v > best ? v : best;
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const uint64_t o = __shfl_xor(best, d, 64);
    best = o > best ? o : best;
  }
  if (lane == 0) out[row] = best ? (int64_t)(uint32_t)~(uint32_t)best : 0;
}

// one workgroup per row, 2-byte loads (rows that are not 16-byte aligned)
template <class T>
__global__ __launch_bounds__(AM_THREADS) void argmax_rows_kernel(const uint16_t *__restrict__ x,
                                                                 int64_t cols, int64_t stride,
                                                                 int64_t *__restrict__ out) {
  const int64_t row = blockIdx.x;
  const uint16_t *xr = x + row * stride;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float best = -INFINITY;
  int64_t bi = cols;  // past the end: loses to every real element
  for (int64_t c = tid; c < cols; c += AM_THREADS) {
    const float v = T::lo(xr[c]);
    if (am_better(v, c, best, bi)) {
      best = v;
      bi = c;
    }
  }
  // the order is total, so the reduction order does not change the result
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float ov = __shfl_xor(best, d, 64);
    const int64_t oi = __shfl_xor(bi, d, 64);
    if (am_better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  __shared__ float bv[AM_THREADS / 64];
  __shared__ int64_t bix[AM_THREADS / 64];
  if (lane == 0) {
    bv[w] = best;
    bix[w] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int k = 1; k < AM_THREADS / 64; ++k)
      if (am_better(bv[k], bix[k], best, bi)) {
        best = bv[k];
        bi = bix[k];
      }
    out[row] = bi < cols ? bi : 0;
  }
}

// one workgroup: the step counter is read by every thread before thread 0
// moves it on
__global__ __launch_bounds__(256) void decode_advance_kernel(
    const int32_t *__restrict__ block_tables, int32_t *__restrict__ positions,
    int32_t *__restrict__ context_lens, int32_t *__restrict__ slot_mapping,
    const int64_t *__restrict__ input_ids, int64_t *__restrict__ token_log,
    int32_t *__restrict__ step_counter, int batch, int max_blocks, int block_size,
    int log_capacity) {
  const int step = token_log ? step_counter[0] : 0;
  __syncthreads();
  if (token_log && threadIdx.x == 0) step_counter[0] = step + 1;
  for (int b = threadIdx.x; b < batch; b += blockDim.x) {
    if (token_log && step >= 0 && step < log_capacity)
      token_log[(int64_t)step * batch + b] = input_ids[b];
    const int pos = positions[b] + 1;
    positions[b] = pos;
    context_lens[b] = context_lens[b] + 1;
    const int64_t blk = pos >= 0 ? pos / block_size : -1;
    slot_mapping[b] = blk >= 0 && blk < max_blocks
                          ? block_tables[(int64_t)b * max_blocks + blk] * block_size +
                                pos % block_size
                          : -1;
  }
}

}  // namespace mce

using namespace mce;

extern "C" size_t mce_argmax_rows_workspace_size(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return (size_t)rows * argmax_parts(cols) * sizeof(uint64_t);
}

extern "C" int mce_argmax_rows(int dtype, const void *logits, int64_t rows, int64_t cols,
                               int64_t row_stride, int64_t *out, void *workspace,
                               size_t workspace_bytes, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "mce_argmax_rows: unknown dtype %d", dtype);
  MCE_REQUIRE(rows >= 0 && cols >= 1 && row_stride >= cols, "mce_argmax_rows: bad shape");
  if (rows == 0) return MCE_OK;
  MCE_REQUIRE(logits && out, "mce_argmax_rows: null pointer");
  // one workgroup per row on grid.x without the split
  MCE_REQUIRE(rows < ((int64_t)1 << 31), "mce_argmax_rows: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const size_t need = mce_argmax_rows_workspace_size(rows, cols);
  const bool split = aligned16(logits) && row_stride % 8 == 0 && cols >= 8 &&
                     cols < ((int64_t)1 << 31);
  if (split) {
    // the split puts rows on grid.y
    MCE_REQUIRE(rows < 65536, "mce_argmax_rows: at most 65535 rows of 16-byte aligned logits");
    if (workspace == nullptr || workspace_bytes < need ||
        (reinterpret_cast<uintptr_t>(workspace) & 7) != 0)
      return set_error(MCE_ERR_WORKSPACE,
                       "mce_argmax_rows: an 8-byte aligned workspace of %zu bytes is required "
                       "(%zu given)", need, workspace_bytes);
    const int parts = argmax_parts(cols);
    const dim3 grid((unsigned)parts, (unsigned)rows);
    uint64_t *part = (uint64_t *)workspace;
    if (dtype == MCE_F16)
      argmax_part_kernel<F16T><<<grid, AMP_THREADS, 0, st>>>((const uint16_t *)logits, (int)cols,
                                                             row_stride, parts, part);
    else
      argmax_part_kernel<BF16T><<<grid, AMP_THREADS, 0, st>>>((const uint16_t *)logits, (int)cols,
                                                              row_stride, parts, part);
    argmax_final_kernel<<<(unsigned)rows, 64, 0, st>>>(part, parts, out);
  } else if (dtype == MCE_F16) {
    argmax_rows_kernel<F16T><<<(unsigned)rows, AM_THREADS, 0, st>>>((const uint16_t *)logits, cols,
                                                                    row_stride, out);
  } else {
    argmax_rows_kernel<BF16T><<<(unsigned)rows, AM_THREADS, 0, st>>>((const uint16_t *)logits,
                                                                     cols, row_stride, out);
  }
  return check_launch("mce_argmax_rows");
}

extern "C" int mce_decode_advance(const int32_t *block_tables, int32_t *positions,
                                  int32_t *context_lens, int32_t *slot_mapping,
                                  const int64_t *input_ids, int64_t *token_log,
                                  int32_t *step_counter, int batch, int max_blocks_per_seq,
                                  int block_size, int log_capacity, void *stream) {
  clear_error();
  MCE_REQUIRE(batch >= 0 && max_blocks_per_seq >= 0 && block_size >= 1 && log_capacity >= 0,
              "mce_decode_advance: bad shape");
  if (batch == 0) return MCE_OK;
  MCE_REQUIRE(block_tables && positions && context_lens && slot_mapping,
              "mce_decode_advance: null pointer");
  MCE_REQUIRE(!token_log || (input_ids && step_counter),
              "mce_decode_advance: a token log needs input_ids and step_counter");
  MCE_REQUIRE((int64_t)max_blocks_per_seq * block_size < ((int64_t)1 << 31),
              "mce_decode_advance: block table too wide");
  decode_advance_kernel<<<1, 256, 0, (hipStream_t)stream>>>(
      block_tables, positions, context_lens, slot_mapping, input_ids, token_log, step_counter,
      batch, max_blocks_per_seq, block_size, log_capacity);
  return check_launch("mce_decode_advance");
}
