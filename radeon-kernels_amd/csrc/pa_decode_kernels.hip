// Paged-attention decode for MI355X (gfx950, CDNA4, wave64).
//
// Operator semantics follow the reference fallback
// (src/radeon_kernels/ops/paged_attention/reference.py:7-47) and contract
// (contracts/paged_attention_decode-1.0.json:15-25): one query token per sequence, query head h
// reads KV head h / (Hq / Hkv), token t lives in slot block_tables[b, t / BS] * BS + t % BS,
// tokens t >= context_length are masked, fp32 softmax and accumulation, output rounded to the
// query dtype.  The reference's own kernel (benchmarks/paged_attention/native_paged_attention.hip)
// runs one wave32 per (sequence, query head) serially over the context; this file is a different
// design built for CDNA4:
//
//   pa_partition_kernel  one 256-thread workgroup per (sequence, KV head, head chunk, context
//                        partition).  Each of its 4 waves walks 16-token tiles of the partition.
//                        K rows are copied by global_load_lds DMA into a multi-buffered,
//                        XOR-swizzled per-wave LDS tile and read from there as MFMA A operands
//                        (tokens on M, query heads of the chunk replicated over N); V rows are
//                        fetched as full-row lane-group loads (one token row per 16 lanes).  The
//                        16x16 MFMA accumulator layout puts the score of token 4g+r for query head
//                        (j % GC) in lane 16g+j, register r -- the same tokens that lane group g
//                        holds for V, and exactly the A-operand layout of a second 16x16x32 MFMA
//                        that computes PV, with the V rows as its B operand after two byte permutes
//                        per column block.  The only cross-lane traffic per tile is a
//                        permlane16/32 swap max-reduction.  Every KV byte is read once per
//                        (KV head, head chunk) and shared by all query heads of the chunk.
//   pa_partition_queue_kernel  the same work items on a work queue: as many workgroups as the
//                        device holds at once, each building the call's item map (largest items
//                        first) from the context lengths and taking items from a ticket counter
//                        until none is left.  Only items with tokens are scheduled.  On long GQA
//                        calls at head_dim 128 (pair_kv_heads) one 8-wave workgroup runs two
//                        adjacent KV heads of an item, four waves each, with the same bits.
//   The last workgroup to finish a split sequence's partitions merges them in the same launch
//   (fused form), or
//   pa_reduce_kernel     deterministic fixed-order merge of the per-partition (max, sum, acc)
//                        records.  Skipped for sequences that fit in one partition (the
//                        partition kernel then writes the normalised output itself) and not
//                        launched at all when one partition covers max_blocks * block_size.
//
// Scores are kept in the base-2 domain: x = (q . k) * scale * log2(e), p = exp2(x - m), which is
// exp(q . k * scale - m') by the identity exp(y) = 2^(y * log2 e); v_exp_f32 evaluates 2^x.
//
// This file is compiled once per element type and head_dim (RK_PA_UNIT_ELEMENT = bf16 | fp16,
// RK_PA_UNIT_HEAD_DIM = 64 | 128 | 256); each compilation defines that unit's launcher, declared in
// pa_decode_common.hpp.  The host side (validation, workspace layout, the C ABI) is
// pa_decode_gfx950.hip.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <atomic>
#include <utility>

#include "pa_decode_common.hpp"
#include "rk_paged_attention.h"

#if !defined(RK_PA_UNIT_ELEMENT) || !defined(RK_PA_UNIT_HEAD_DIM)
#error "compile once per unit: -DRK_PA_UNIT_ELEMENT=bf16|fp16 -DRK_PA_UNIT_HEAD_DIM=64|128|256"
#endif

namespace rk_pa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------------------------
// Element traits: 16-bit storage, fp32 math.
struct Bf16 {
  static __device__ __forceinline__ float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return __builtin_bit_cast(float, w & 0xffff0000u);
  }
  static __device__ __forceinline__ uint16_t store(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  }
  // Two values rounded to the element type, x in the low half.
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    return static_cast<uint32_t>(store(x)) | (static_cast<uint32_t>(store(y)) << 16);
  }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

struct Fp16 {
  static __device__ __forceinline__ float lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  }
  static __device__ __forceinline__ uint16_t store(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    return static_cast<uint32_t>(store(x)) | (static_cast<uint32_t>(store(y)) << 16);
  }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// ---------------------------------------------------------------------------------------------
// Cross-lane helpers (wave64).
__device__ __forceinline__ uint32_t bits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float fbits(uint32_t x) { return __builtin_bit_cast(float, x); }

// DPP: quad_perm broadcast of quad lane H to all four lanes of each quad.
template <int H>
__device__ __forceinline__ float quad_bcast(float x) {
  return fbits(__builtin_amdgcn_update_dpp(0, bits(x), H * 0x55, 0xF, 0xF, false));
}

// ds_swizzle in bit mode: lane H of each 8-lane group to all eight (lane' = (lane & 0x18) | H, within
// each 32-lane half).  No LDS memory is touched.
template <int H>
__device__ __forceinline__ float oct_bcast(float x) {
  return fbits(__builtin_amdgcn_ds_swizzle(bits(x), 0x18 | (H << 5)));
}
template <int... H>
__device__ __forceinline__ void oct_all(float x, float* out, std::integer_sequence<int, H...>) {
  ((out[H] = oct_bcast<H>(x)), ...);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return fbits(__builtin_amdgcn_update_dpp(0, bits(x), CTRL, 0xF, 0xF, false));
}

// v_permlane16_swap exchanges odd 16-lane rows of its first operand with even rows of the second;
// feeding the same value to both yields {x[l & ~16], x[l | 16]} per lane, so combining the pair
// gives the xor-16 reduction in every lane.  v_permlane32_swap does the same for the two halves.
__device__ __forceinline__ float max_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(bits(x), bits(x), false, false);
  return fmaxf(fbits(r[0]), fbits(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(bits(x), bits(x), false, false);
  return fmaxf(fbits(r[0]), fbits(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(bits(x), bits(x), false, false);
  return fbits(r[0]) + fbits(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(bits(x), bits(x), false, false);
  return fbits(r[0]) + fbits(r[1]);
}

// Sum over the 16 lanes of each DPP row; every lane of the row receives the row total.
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  x += dpp<0x140>(x);  // row_mirror
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K and V cache rows are read exactly once per launch, so their loads carry the non-temporal cache
// policy (nt): a read-only probe of this access pattern (256-byte rows of shuffled 32 KB blocks, 4.8
// GB) streamed at 6.19 TB/s with it against 5.80 TB/s without.
constexpr int kCpolNonTemporal = 2;  // the nt bit of the gfx940-family cache-policy field

// global_load_lds_dwordx4: each lane's 16 bytes at `src` land in LDS at `lds_base` + 16 * lane
// (lds_base must be wave-uniform).  Completion is tracked by the wave's memory counter.  Kept in a
// device function so the host compilation pass never sees the target builtin.
__device__ __forceinline__ void dma_to_lds16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, lds_base, 16, 0, kCpolNonTemporal);
}

// LDS reads that complete before they return (ds_read + s_waitcnt lgkmcnt(0) in one statement).
// The compiler places a conservative vmcnt(0) wait in front of every LDS read it emits while an
// LDS-DMA is outstanding, since it cannot tell which LDS bytes the DMA writes; that wait would stall
// on the loads of tiles still in flight.  The kernel issues these reads only after its own explicit
// memory-counter wait has covered the DMA that wrote the bytes being read.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  typedef const __attribute__((address_space(3))) char lds_char;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char*)(p)));
}

__device__ __forceinline__ int lds_read_i32_sync(uint32_t addr) {
  int v;
  __asm__ __volatile__("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

template <int OFFSET>
__device__ __forceinline__ void lds_read2x16_sync(u32x4& a, u32x4& b, uint32_t aa, uint32_t ab) {
  __asm__ __volatile__(
      "ds_read_b128 %0, %2 offset:%4\n\t"
      "ds_read_b128 %1, %3 offset:%4\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a), "=&v"(b)
      : "v"(aa), "v"(ab), "i"(OFFSET)
      : "memory");
}

template <int OFFSET>
__device__ __forceinline__ void lds_read4x16_sync(u32x4& a, u32x4& b, u32x4& c, u32x4& d, uint32_t aa,
                                                  uint32_t ab, uint32_t ac, uint32_t ad) {
  __asm__ __volatile__(
      "ds_read_b128 %0, %4 offset:%8\n\t"
      "ds_read_b128 %1, %5 offset:%8\n\t"
      "ds_read_b128 %2, %6 offset:%8\n\t"
      "ds_read_b128 %3, %7 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d)
      : "v"(aa), "v"(ab), "v"(ac), "v"(ad), "i"(OFFSET)
      : "memory");
}

// Workgroup barrier that publishes this wave's LDS writes but, unlike __syncthreads, does not wait
// for its outstanding global loads (the K/V loads already in flight stay in flight).
__device__ __forceinline__ void lds_barrier() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkmcnt0);
  __builtin_amdgcn_s_barrier();
  __asm__ __volatile__("" ::: "memory");
}

template <bool B>
struct Flag {
  static constexpr bool value = B;
};

template <int N>
struct Int {
  static constexpr int value = N;
};

// f(Int<0>{}), ..., f(Int<N - 1>{}) in order: a loop whose index is a compile-time constant in the
// body, so that register arrays indexed by it stay in registers.
template <class F, int... K>
__device__ __forceinline__ void unroll_each(F&& f, std::integer_sequence<int, K...>) {
  (f(Int<K>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void unroll(F&& f) {
  unroll_each(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ int64_t load_index(const void* base, int64_t i, bool is64) {
  return is64 ? static_cast<const int64_t*>(base)[i]
              : static_cast<int64_t>(static_cast<const int32_t*>(base)[i]);
}

// The two 32-bit words of an index element, loaded without branching on the index type (for int32
// both words are the element itself); decoded by index_value once the loads have landed.  Keeps
// independent index loads in flight together instead of waiting on each at an int32/int64 merge.
struct RawIndex {
  uint32_t lo, hi;
};
__device__ __forceinline__ RawIndex load_raw_index(const void* base, int64_t i, bool is64) {
  const uint32_t* words = static_cast<const uint32_t*>(base);
  const int64_t at = is64 ? 2 * i : i;
  return RawIndex{words[at], words[is64 ? at + 1 : at]};
}
__device__ __forceinline__ int64_t index_value(RawIndex r, bool is64) {
  return is64 ? static_cast<int64_t>((static_cast<uint64_t>(r.hi) << 32) | r.lo)
              : static_cast<int64_t>(static_cast<int32_t>(r.lo));
}

__device__ __forceinline__ int64_t clamped_context(const Params& p, int b) {
  const int64_t max_ctx = static_cast<int64_t>(p.max_blocks) << p.bs_log2;
  const int64_t ctx = load_index(p.context_lengths, b, p.index_is64 != 0);
  return ctx < max_ctx ? ctx : max_ctx;
}

// ---------------------------------------------------------------------------------------------
// Partition merge of one (sequence, query head) row by one wave.  The global maximum comes from a
// wave-wide max over the partition maxima; each lane then owns one record's weight
// exp2(m_i - M), the sum is a wave-wide sum of l_i * weight, and the accumulator columns are
// merged in partition-index order, a group of records at a time with all their loads issued
// together.  Fixed order and fixed grouping make the result deterministic, and the reduce kernel
// and the fused epilogue of the partition kernel run this same code, so both give bit-identical
// outputs.
//
// Records cross XCDs (each XCD has its own L2).  They are stored with agent-scope atomic stores
// (write-through to the device coherence point, no dirty L2 lines) and, inside the fused epilogue,
// read with agent-scope atomic loads (fetched from the coherence point, never from a stale line of
// this XCD's L2).  Neither needs the whole-L2 write-back or invalidate that an agent-scope fence
// performs; ordering between the stores and the arrival counter comes from waiting for the stores'
// acknowledgements before the counter is incremented.
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) x = fmaxf(x, __shfl_xor(x, offset));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) x += __shfl_xor(x, offset);
  return x;
}

__device__ __forceinline__ void store_record(float* ptr, float x) {
  __hip_atomic_store(ptr, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool COHERENT>
__device__ __forceinline__ float load_record(const float* ptr) {
  if constexpr (COHERENT) {
    return __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    return *ptr;  // after a kernel boundary: the launch order already makes the records visible
  }
}

template <class E, int D, bool COHERENT>
__device__ __forceinline__ void merge_partitions(const Params& p, int64_t row, int np, int lane) {
  constexpr int PER_LANE = D / kWave;
  constexpr int GROUP = 32 / PER_LANE;  // 32 accumulator loads in flight per lane; divides 64
  const float* ml = p.ws_ml + row * p.num_partitions * 2;
  const float* acc = p.ws_acc + row * p.num_partitions * D;
  const float neg_inf = -__builtin_inff();
  // Accumulator columns of records i0 .. i0 + GROUP - 1 (an index past np re-reads the last record;
  // its weight is 0 and fmaf(v, 0, A) == A, so the padding leaves the sum unchanged).
  auto load_group = [&](float (&vals)[GROUP][PER_LANE], int i0) {
#pragma unroll
    for (int u = 0; u < GROUP; ++u) {
      const int64_t i = min(i0 + u, np - 1);
#pragma unroll
      for (int c = 0; c < PER_LANE; ++c) vals[u][c] = load_record<COHERENT>(acc + i * D + lane + c * kWave);
    }
  };

  // One memory round: lane j's own (max, sum) record j and the first group of accumulators.
  float m_lane = neg_inf, l_lane = 0.0f;
  if (lane < np) {
    m_lane = load_record<COHERENT>(ml + 2 * lane);
    l_lane = load_record<COHERENT>(ml + 2 * lane + 1);
  }
  float vals[GROUP][PER_LANE];
  load_group(vals, 0);
  float M = fmaxf(neg_inf, m_lane);
  for (int i = lane + kWave; i < np; i += kWave) M = fmaxf(M, load_record<COHERENT>(ml + 2 * i));
  M = wave_max(M);

  // Records in chunks of 64: lane j computes the weight of record c0 + j (0 past np), the sum
  // accumulates per lane, and the accumulator columns take the weights in record order by
  // broadcast from the owning lane.
  float L = 0.0f;
  float A[PER_LANE];
#pragma unroll
  for (int c = 0; c < PER_LANE; ++c) A[c] = 0.0f;
  for (int c0 = 0; c0 < np; c0 += kWave) {
    float mi = m_lane, li = l_lane;
    if (c0 > 0) {
      mi = neg_inf;
      li = 0.0f;
      if (c0 + lane < np) {
        mi = load_record<COHERENT>(ml + 2 * (c0 + lane));
        li = load_record<COHERENT>(ml + 2 * (c0 + lane) + 1);
      }
    }
    const float f = (mi == neg_inf) ? 0.0f : fast_exp2(mi - M);
    L += (mi == neg_inf) ? 0.0f : li * f;
    const int n = min(kWave, np - c0);
    for (int u0 = 0; u0 < n; u0 += GROUP) {
      if (c0 + u0 > 0) load_group(vals, c0 + u0);
#pragma unroll
      for (int u = 0; u < GROUP; ++u) {
        const float fu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), u0 + u));
#pragma unroll
        for (int c = 0; c < PER_LANE; ++c) A[c] = fmaf(vals[u][c], fu, A[c]);
      }
    }
  }
  L = wave_sum(L);
  const float inv = 1.0f / L;
#pragma unroll
  for (int c = 0; c < PER_LANE; ++c) p.out[row * D + lane + c * kWave] = E::store(A[c] * inv);
}

// ---------------------------------------------------------------------------------------------
// Partition reduce: one wave per (sequence, query head), for rows whose sequence spans several
// partitions (the partition kernel writes the others itself).
template <class E, int D>
__global__ __launch_bounds__(kThreads) void pa_reduce_kernel(Params p) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= static_cast<int64_t>(p.batch) * p.query_heads) return;
  const int b = static_cast<int>(row / p.query_heads);
  const int64_t ctx = clamped_context(p, b);
  if (ctx <= 0) return;  // written by the partition kernel
  // The partition size the queue kernel ran; a stored value outside [partition_tokens,
  // grow_max_tokens] is not one it can run, and the call's own size keeps the reads in the records.
  int P = p.partition_tokens;
  if (p.grown != nullptr) {
    const int g = static_cast<int>(*p.grown);
    if (g > P && g <= p.grow_max_tokens) P = g;
  }
  const int np = static_cast<int>((ctx + P - 1) / P);
  if (np <= 1) return;   // written by the partition kernel
  merge_partitions<E, D, false>(p, row, np, lane);
}

// ---------------------------------------------------------------------------------------------
// Split-K partition kernel.
//   E       element traits (Bf16 / Fp16)
//   D       head_dim (64, 128, 256)
//   GC      query heads handled per workgroup (1, 2, 4, 8); all share one KV head.  Groups of 8 or
//           more run in chunks of 8 at head_dim 64 and 128: each KV row is read once per 8 query
//           heads.  With PV on fp32 FMAs the 8-head accumulators take 304-308 registers at head_dim
//           128 (one wave per SIMD) and the chunk still measured 1.32-1.67x faster than two chunks
//           of 4; with PV on MFMA a lane holds 4 of the 8 heads' accumulators and the chunk runs at
//           two waves per SIMD.  At head_dim 64 the 8-head chunk measured 1.6-1.75x faster than
//           two chunks of 4 (128x8 and 64x8 layouts).  At head_dim 256 it is built with PV on MFMA
//           only (with PV on fp32 FMAs its accumulators spill)
//   QK_MFMA QK^T on MFMA (true) or on fp32 FMAs + DPP row sums (false)
//   PV_MFMA PV on MFMA as well (QK_MFMA only): the probabilities leave the QK^T MFMA in exactly the
//           A-operand layout of a 16x16x32 MFMA (lane 16g + j: score column j, tokens 4g..4g+3), and
//           the V rows a lane holds (tokens 4g..4g+3, columns j*VEC .. j*VEC + VEC - 1) give the B
//           operand of output column block e (columns j*VEC + e) with two byte permutes, so no data
//           moves between lanes.  Each probability enters as a rounded high part and its residual
//           (k 0..3 and 4..7 of the lane's 8 k-slots, V repeated), which keeps it to about 2^-16
//           relative: the product is as accurate as the fp32 FMAs it replaces to within the fp32
//           accumulation.  Output row 4g + i is score column 4g + i, query head (4g + i) % GC.
//   UB      block_size >= 16: every 16-aligned tile lies inside one cache block, so the block id is
//           wave-uniform and addresses are a scalar base plus fixed 32-bit per-lane offsets
//   AP      append-and-decode: each sequence's new token (position ctx - 1) is read from new_k /
//           new_v instead of the cache, and the workgroup whose partition holds it (head chunk 0)
//           stores its KV head's rows into the token's cache slot.  No other workgroup of the launch
//           reads that slot (its block belongs to this sequence's tail), so nothing waits for the
//           store; the next launch sees it.  MFMA variant only.
//
// MFMA variants' data path per 16-token tile and wave:
//   K: global_load_lds_dwordx4 straight into a per-wave LDS slot.  Each DMA instruction moves
//      whole cache rows (coalesced); lane l fetches chunk (l % CPR) ^ (row & SWZ) of its row, so
//      the hardware's lane-contiguous LDS write leaves the tile XOR-swizzled and the MFMA operand
//      read (token j, chunk 4i+g) is bank-conflict free.
//   V: 16-byte register loads, one token row per 16-lane group (rows 4g..4g+3).
//   Pipeline: DEPTH tiles are in flight ahead of the one being computed (DEPTH + 1 register tiles
//   and LDS K slots rotate).  Step n: wait until tile n has landed -> issue tile n + DEPTH ->
//   read K(n) from LDS -> MFMA -> softmax -> PV(n) (MFMA, or fp32 FMAs when PV_MFMA is false).
//
// partition_item is one work item (sequence b, head slot = KV head * head_chunks + head chunk,
// partition part) run by the whole workgroup (tid = threadIdx.x); the two kernels below differ only
// in how they hand out work items.  at_epilogue() runs in every wave once the item's loads have all
// landed, at the start of its epilogue (not for an item that ends early: an empty context or a
// partition past it); memory operations it issues are waited for only where their results are used.
template <class E, int D, int GC, bool QK_MFMA, bool PV_MFMA, bool UB, bool AP, int KVP, class Epilogue>
__device__ __attribute__((always_inline)) inline void partition_item(const Params& p, const int tid, int b, int hslot,
                                                                     int part, const int P, Epilogue&& at_epilogue) {
  static_assert(!AP || QK_MFMA, "append-and-decode is built for the MFMA variants");
  static_assert(!PV_MFMA || QK_MFMA, "PV on MFMA takes its A operand from the QK^T MFMA's score layout");
  static_assert(KVP == 1 || KVP == 2, "one or two KV heads per workgroup");
  // KVP KV heads per workgroup, each run by its own group of kWaves waves exactly as a one-head
  // workgroup runs it (same tiles, same merge order, so the same bits); the groups share the
  // partition's block-table slice.
  constexpr int NWAVES = kWaves * KVP;
  constexpr int NTHREADS = kThreads * KVP;
  constexpr int KSTEPS = D / 32;       // MFMA k-steps; also DMA instructions per K tile
  constexpr int VEC = D / 16;          // elements of a token row per lane (row = 16 lanes)
  constexpr int VW = VEC / 2;          // 32-bit words per lane per token row
  constexpr int CPR = D / 8;           // 16-byte chunks per cache row (one token, one KV head)
  constexpr int RPI = kWave / CPR;     // cache rows per DMA instruction
  constexpr int SWZ = CPR - 1 < 15 ? CPR - 1 : 15;  // chunk swizzle mask
  constexpr int KTILE16 = kTile * CPR; // 16-byte units of one staged K tile
  static_assert(GC == 1 || GC == 2 || GC == 4 || GC == 8, "head chunk must be 1, 2, 4 or 8");
  static_assert(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
  static_assert(KTILE16 == KSTEPS * kWave, "one DMA instruction per MFMA k-step");
  // Tiles in flight ahead of the current one: two when K is staged in LDS, blocks hold whole tiles
  // and head_dim <= 128; one for head_dim 256 (K slots twice as large, register file already mostly
  // used), for the VALU variant (K rows held in registers: a third tile would push it to one wave
  // per SIMD) and for blocks smaller than a tile (per-lane block-table reads in LDS).
  constexpr int DEPTH = (QK_MFMA && UB && D != 256) ? 2 : 1;
  constexpr int SLOTS = DEPTH + 1;
  static_assert(UB || DEPTH == 1, "tiles past the first need their block ids before the table is staged");
  // Vector memory instructions one tile issues (K DMA or K rows, then V rows): the unit of the
  // explicit memory-counter waits.
  constexpr int ROW_LOADS = 4 * (VW >= 4 ? VW / 4 : 1);
  constexpr int TILE_OPS = (QK_MFMA ? KSTEPS : ROW_LOADS) + ROW_LOADS;

  // The K staging slots and, after the main loop, the per-wave partial accumulators share one
  // LDS buffer (a barrier separates the two uses).
  constexpr int SLOT_BYTES = KTILE16 * 16;
  constexpr int K_STAGE_BYTES = QK_MFMA ? NWAVES * SLOTS * SLOT_BYTES : 0;
  constexpr int ACC_BYTES = NWAVES * GC * D * 4;
  constexpr int RAW_BYTES = K_STAGE_BYTES > ACC_BYTES ? K_STAGE_BYTES : ACC_BYTES;
  __shared__ __attribute__((aligned(16))) unsigned char s_raw[RAW_BYTES];
  __shared__ int s_table[kMaxSliceBlocks];
  __shared__ float s_m[NWAVES][GC];
  __shared__ float s_l[NWAVES][GC];
  __shared__ int s_last;

  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wl = wave % kWaves;    // wave within its KV head's group
  const int kvsub = wave / kWaves;  // which of the workgroup's KV heads
  const int lane = tid & 63;
  const int g = lane >> 4;   // lane group: owns tokens 4g..4g+3 of every tile (V / scores)
  const int j = lane & 15;   // lane in group: token j of the tile for K (MFMA), V column block
  u32x4* const s_k = reinterpret_cast<u32x4*>(s_raw) + wave * SLOTS * KTILE16;
  float(*const s_acc)[GC][D] = reinterpret_cast<float(*)[GC][D]>(s_raw);

  const int heads_per_seq = (p.kv_heads / KVP) * p.head_chunks;  // work items per (sequence, partition)
  const int kvh0 = (hslot / p.head_chunks) * KVP;                // the workgroup's first KV head
  const int kvh = kvh0 + kvsub;                                   // this wave's KV head
  const int chunk = hslot % p.head_chunks;
  const int head0 = kvh * p.group + chunk * GC;  // first query head of this wave's chunk
  const int heads_here = min(GC, p.group - chunk * GC);

  // Prologue.  Every load that does not depend on the context length -- the context length
  // itself, this partition's block-table slice, the query and (uniform-block path) the block ids of
  // the wave's first tiles -- is issued together, so the workgroup waits one memory latency, not
  // three, before it sends out its first K/V loads.
  const int lb = p.bs_log2;
  const int bs_mask = (1 << lb) - 1;
  const int p0 = part * P;
  const int blk0 = p0 >> lb;
  // Entries of the partition's blocks that exist in the table row (<= 0 when the partition starts
  // past the row; the context-length check below then ends the workgroup).
  const int slice = min(((p0 + P - 1) >> lb) - blk0 + 1, p.max_blocks - blk0);
  const int64_t table_row = static_cast<int64_t>(b) * p.max_blocks + blk0;
  const bool is64 = p.index_is64 != 0;
  const RawIndex ctx_raw = load_raw_index(p.context_lengths, b, is64);
  static_assert(2 * NTHREADS >= kMaxSliceBlocks, "two table entries per thread cover a partition's slice");
  RawIndex ids[2] = {{~0u, ~0u}, {~0u, ~0u}};  // entries tid and tid + NTHREADS (a slice has <= 512)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + i * NTHREADS;
    if (idx < slice) ids[i] = load_raw_index(p.block_tables, table_row + idx, is64);
  }

  // Append: lanes [0, CPR) of each KV head's first wave hold one 16-byte chunk of the new token's K row,
  // lanes [CPR, 2 CPR) of its V row, loaded with the prologue.
  const int64_t new_row = (static_cast<int64_t>(b) * p.kv_heads + kvh) * D;
  u32x4 ap_chunk = {0u, 0u, 0u, 0u};
  if constexpr (AP) {
    if (wl == 0 && lane < 2 * CPR) {
      const uint16_t* src = (lane < CPR ? p.new_k : p.new_v) + new_row + (lane % CPR) * 8;
      ap_chunk = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
    }
  }

  // Query operands.
  const int64_t q_row0 = static_cast<int64_t>(b) * p.query_heads + head0;
  const int my_head = j % GC;  // head of the scores this lane holds
  u32x4 qB[QK_MFMA ? KSTEPS : 1];
  float qf[QK_MFMA ? 1 : GC][QK_MFMA ? 1 : VEC];
  if constexpr (QK_MFMA) {
    // B operand of S^T = K Q^T: column n <-> query head (n % GC), k-chunk (4i + g) of 8 elements.
    const bool ok = my_head < heads_here;
    const uint16_t* src = p.q + (q_row0 + my_head) * D + g * 8;
#pragma unroll
    for (int i = 0; i < KSTEPS; ++i) {
      qB[i] = ok ? *reinterpret_cast<const u32x4*>(src + i * 32) : u32x4{0, 0, 0, 0};
    }
  } else {
#pragma unroll
    for (int h = 0; h < GC; ++h) {
      const bool ok = h < heads_here;
      const uint16_t* src = p.q + (q_row0 + h) * D + j * VEC;
#pragma unroll
      for (int w = 0; w < VW; ++w) {
        const uint32_t word = ok ? reinterpret_cast<const uint32_t*>(src)[w] : 0u;
        qf[h][2 * w] = E::lo(word);
        qf[h][2 * w + 1] = E::hi(word);
      }
    }
  }

  // Block ids of this wave's first DEPTH tiles (tokens p0 + 16 * wl + 64 * n), read straight from
  // the table so they can be issued before the staged slice is visible to the wave.
  RawIndex first_raw[DEPTH];
#pragma unroll
  for (int n = 0; n < DEPTH; ++n) {
    first_raw[n] = RawIndex{~0u, ~0u};
    const int idx = ((p0 + wl * kTile + n * kWaves * kTile) >> lb) - blk0;
    if (UB && idx < slice) first_raw[n] = load_raw_index(p.block_tables, table_row + idx, is64);
  }
  auto valid_block = [&](RawIndex r) -> int {
    const int64_t id = index_value(r, is64);
    return (id >= 0 && id < p.num_blocks) ? static_cast<int>(id) : -1;
  };

  const int64_t max_ctx = static_cast<int64_t>(p.max_blocks) << lb;
  const int64_t ctx_len = index_value(ctx_raw, is64);
  const int64_t ctx = ctx_len < max_ctx ? ctx_len : max_ctx;
  if (ctx <= 0) {
    // Softmax over an empty set: NaN, as the fallback produces.  Partition 0 owns the output.
    if (part == 0) {
      for (int idx = tid; idx < KVP * heads_here * D; idx += NTHREADS) {
        const int kv = KVP == 1 ? 0 : idx / (heads_here * D);
        const int hd = KVP == 1 ? idx : idx - kv * heads_here * D;
        const int h = hd / D, d = hd % D;
        const int head = (kvh0 + kv) * p.group + chunk * GC + h;
        p.out[(static_cast<int64_t>(b) * p.query_heads + head) * D + d] = E::store(__builtin_nanf(""));
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  const int np = static_cast<int>((ctx + P - 1) / P);
  if (part >= np) {
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  const int p_end = static_cast<int>(min(static_cast<int64_t>(p0 + P), ctx));
  // Append: the new token's position, and whether this partition holds it (the last one does).  A
  // context length past the table puts the new token outside it: it is neither stored nor read, and
  // the partitions cover the table's tokens as they do without an append.
  const int ap_pos = static_cast<int>(ctx - 1);
  const bool ap_here = AP && ctx_len <= max_ctx && ap_pos >= p0 && ap_pos < p_end;

  // Stage this partition's block-table slice in LDS (-1 marks ids outside [0, num_blocks)).  It is
  // made visible by the barrier in front of the main loop.
  const int nblk = ((p_end - 1) >> lb) - blk0 + 1;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + i * NTHREADS;
    if (idx < nblk) s_table[idx] = valid_block(ids[i]);
  }

  const uint16_t* __restrict__ kbase = p.k + static_cast<int64_t>(kvh) * D;
  const uint16_t* __restrict__ vbase = p.v + static_cast<int64_t>(kvh) * D;

  struct Tile {
    uint32_t kr[QK_MFMA ? 1 : 4][QK_MFMA ? 1 : VW];  // VALU variant: K rows like V
    uint32_t v[4][VW];
    uint32_t valid;  // bit r: token t0 + 4g + r is inside the partition and its block is valid
    bool full;       // wave-uniform: all 16 tokens valid (no masking needed)
  };

  // Loads are unconditional and always in bounds: a token past the partition end, or one whose
  // block id is invalid, reads a row of block 0 (or of the tile's block) instead and its data is
  // discarded after the load (score -> -inf, V row -> 0).  Branch-free loads keep the wave's
  // memory counter exact, so the next tile's loads stay in flight while the current one is used.
  const int last = p_end - 1;
  auto block_of = [&](int t) -> int { return s_table[(min(t, last) >> lb) - blk0]; };
  auto row_base = [&](int pb, int t) -> int64_t {
    return static_cast<int64_t>(pb < 0 ? 0 : pb) * p.block_stride +
           static_cast<int64_t>(t & bs_mask) * p.row_stride;
  };

  // Per-lane element offsets relative to a tile's first row (uniform-block path); the host
  // guarantees 16 * row_stride fits in 31 bits.
  const int32_t row_stride32 = static_cast<int32_t>(p.row_stride);
  int32_t v_lane_off[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v_lane_off[r] = (4 * g + r) * row_stride32 + j * VEC;
  const int dma_row = lane / CPR;  // row (within RPI) a lane moves in each K DMA instruction
  const int dma_pos = lane % CPR;  // its 16-byte position in the staged row
  int32_t kdma_off[QK_MFMA ? KSTEPS : 1];
  uint32_t kread[QK_MFMA ? KSTEPS : 1];  // LDS byte address of this lane's operand chunk, slot 0
  if constexpr (QK_MFMA) {
#pragma unroll
    for (int n = 0; n < KSTEPS; ++n) {
      const int row = RPI * n + dma_row;
      kdma_off[n] = row * row_stride32 + ((dma_pos ^ (row & SWZ)) << 3);
    }
    const uint32_t k_lds = lds_address(s_k);
#pragma unroll
    for (int i = 0; i < KSTEPS; ++i) kread[i] = k_lds + 16u * (j * CPR + ((4 * i + g) ^ (j & SWZ)));
  }
  const uint32_t table_lds = lds_address(s_table);

  auto load_v_rows = [&](uint32_t (&dst)[4][VW], const uint16_t* const src[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (VW == 2) {
        const u32x2 x = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src[r]));
        dst[r][0] = x[0];
        dst[r][1] = x[1];
      } else {
#pragma unroll
        for (int w4 = 0; w4 < VW / 4; ++w4) {
          const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src[r] + w4 * 8));
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[r][w4 * 4 + e] = x[e];
        }
      }
    }
  };

  // Issue every load of the tile starting at token t0: K into LDS slot `slot` (MFMA variant) or
  // registers (VALU variant), V into registers.
  // Uniform-block form: `pb` is the tile's block id (-1 when invalid).
  auto issue_tile_block = [&](Tile& tile, int slot, int t0, int pb) __attribute__((always_inline)) {
    const uint16_t* vrow[4];
    const uint16_t* krow[4];
    if constexpr (UB) {
      const bool block_ok = pb >= 0;
      const int64_t base = static_cast<int64_t>(block_ok ? pb : 0) * p.block_stride +
                           static_cast<int64_t>(t0 & bs_mask) * p.row_stride;
      tile.full = block_ok && t0 + kTile <= p_end;
      tile.valid = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) tile.valid |= (block_ok && t0 + 4 * g + r < p_end) ? (1u << r) : 0u;
      if constexpr (AP) {
        // The new token's tile (a wave-uniform branch, taken once per sequence and KV head): its row
        // comes from new_k / new_v through per-lane address selects.  It issues the same loads in the
        // same order as the common path below, which keeps its scalar-base addressing.
        if (ap_here && ap_pos >= t0 && ap_pos < t0 + kTile) {
          u32x4* dst = s_k + slot * KTILE16;
#pragma unroll
          for (int n = 0; n < KSTEPS; ++n) {
            const int row = RPI * n + dma_row;
            const uint16_t* src = t0 + row == ap_pos ? p.new_k + new_row + ((dma_pos ^ (row & SWZ)) << 3)
                                                     : kbase + base + kdma_off[n];
            dma_to_lds16(src, dst + n * kWave);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r)
            vrow[r] = t0 + 4 * g + r == ap_pos ? p.new_v + new_row + j * VEC : vbase + base + v_lane_off[r];
          load_v_rows(tile.v, vrow);
          return;
        }
      }
      if constexpr (QK_MFMA) {
        const uint16_t* kb = kbase + base;
        u32x4* dst = s_k + slot * KTILE16;
#pragma unroll
        for (int n = 0; n < KSTEPS; ++n)
          dma_to_lds16(kb + kdma_off[n], dst + n * kWave);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vrow[r] = vbase + base + v_lane_off[r];
        krow[r] = kbase + base + v_lane_off[r];
      }
    } else {
      tile.full = false;
      tile.valid = 0;
      if constexpr (QK_MFMA) {
        u32x4* dst = s_k + slot * KTILE16;
#pragma unroll
        for (int n = 0; n < KSTEPS; ++n) {
          const int row = RPI * n + dma_row;
          const int t = t0 + row;
          const uint16_t* src = kbase + row_base(block_of(t), t) + ((dma_pos ^ (row & SWZ)) << 3);
          if constexpr (AP) {
            if (ap_here && t == ap_pos) src = p.new_k + new_row + ((dma_pos ^ (row & SWZ)) << 3);
          }
          dma_to_lds16(src, dst + n * kWave);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + 4 * g + r;
        const int pb = block_of(t);
        tile.valid |= (t < p_end && pb >= 0) ? (1u << r) : 0u;
        vrow[r] = vbase + row_base(pb, t) + j * VEC;
        krow[r] = kbase + row_base(pb, t) + j * VEC;
        if constexpr (AP) {
          if (ap_here && t == ap_pos) vrow[r] = p.new_v + new_row + j * VEC;
        }
      }
    }
    if constexpr (!QK_MFMA) load_v_rows(tile.kr, krow);  // K rows of masked tokens need no zeroing
    load_v_rows(tile.v, vrow);
  };
  auto issue_tile = [&](Tile& tile, int slot, int t0) __attribute__((always_inline)) {
    int pb = -1;
    if constexpr (UB) {
      const int t_tab = min(t0, last);  // a tile past the partition end reads a valid table entry
      pb = __builtin_amdgcn_readfirstlane(lds_read_i32_sync(table_lds + 4u * ((t_tab >> lb) - blk0)));
    }
    issue_tile_block(tile, slot, t0, pb);
  };

  // Online-softmax state.  m_own / l_own belong to head my_head (identical across lane groups
  // after the per-tile reductions).  VALU PV: acc[h][e] is head h, column j*VEC + e, over this lane
  // group's tokens.  MFMA PV: accm[e][i] is head (4g + i) % GC, column j*VEC + e, over all tokens.
  const float neg_inf = -__builtin_inff();
  float m_own = neg_inf;
  float l_own = 0.0f;
  float acc[PV_MFMA ? 1 : GC][PV_MFMA ? 1 : VEC];
  f32x4 accm[PV_MFMA ? VEC : 1];
#pragma unroll
  for (int h = 0; h < (PV_MFMA ? 1 : GC); ++h)
#pragma unroll
    for (int e = 0; e < (PV_MFMA ? 1 : VEC); ++e) acc[h][e] = 0.0f;
#pragma unroll
  for (int e = 0; e < (PV_MFMA ? VEC : 1); ++e) accm[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Scores of tokens 4g..4g+3 for head my_head, base-2 scaled, -inf where masked.  Branch-free
  // (the full-tile shortcut is a select) so no control flow sits between the tile's wait and its use.
  auto qk_phase = [&](const Tile& tile, auto slot_tag, float (&x)[4]) __attribute__((always_inline)) {
    const bool FULL = tile.full;
    if constexpr (QK_MFMA) {
      constexpr int OFFSET = decltype(slot_tag)::value * SLOT_BYTES;
      u32x4 kop[KSTEPS];
      if constexpr (KSTEPS == 2) {
        lds_read2x16_sync<OFFSET>(kop[0], kop[1], kread[0], kread[1]);
      } else {
#pragma unroll
        for (int i = 0; i < KSTEPS; i += 4)
          lds_read4x16_sync<OFFSET>(kop[i], kop[i + 1], kop[i + 2], kop[i + 3], kread[i], kread[i + 1],
                                    kread[i + 2], kread[i + 3]);
      }
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < KSTEPS; ++i) s = E::mfma(kop[i], qB[i], s);
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = (FULL || ((tile.valid >> r) & 1u)) ? s[r] * p.scale_log2e : neg_inf;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float kf[VEC];
#pragma unroll
        for (int w = 0; w < VW; ++w) {
          kf[2 * w] = E::lo(tile.kr[r][w]);
          kf[2 * w + 1] = E::hi(tile.kr[r][w]);
        }
        float mine = 0.0f;
#pragma unroll
        for (int h = 0; h < GC; ++h) {
          float dot = 0.0f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) dot = fmaf(qf[h][e], kf[e], dot);
          dot = row_sum16(dot);
          mine = (h == my_head) ? dot : mine;
        }
        x[r] = (FULL || ((tile.valid >> r) & 1u)) ? mine * p.scale_log2e : neg_inf;
      }
    }
  };

  auto pv_phase = [&](const Tile& tile, const float (&x)[4], auto full_tag) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_tag)::value;
    // Tile maximum for my_head over the 16 tokens (4 registers x 4 lane groups).
    float tmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    tmax = max_xor16(tmax);
    tmax = max_xor32(tmax);
    const float m_new = fmaxf(m_own, tmax);
    if (__builtin_amdgcn_ballot_w64(m_new > m_own) != 0) {
      // Rescale all heads' accumulators: alpha_h = 2^(m_old_h - m_new_h), broadcast per quad.
      const float alpha_own = fast_exp2(m_own - m_new);  // 0 when m_own = -inf
      if constexpr (PV_MFMA) {
        // Accumulator row i of this lane holds head (4g + i) % GC: its factor comes from the lane of
        // this lane's quad (8-head chunks: 8-lane group) that holds that head's scores.
        float a4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (GC == 1) {
            a4[i] = alpha_own;
          } else if constexpr (GC == 8) {
            const int src = (lane & ~7) | ((lane >> 2) & 4) | i;  // head 4 (g & 1) + i of the group
            a4[i] = fbits(__builtin_amdgcn_ds_bpermute(src << 2, bits(alpha_own)));
          } else {
            a4[i] = i % GC == 0 ? quad_bcast<0>(alpha_own)
                    : i % GC == 1 ? quad_bcast<1>(alpha_own)
                    : i % GC == 2 ? quad_bcast<2>(alpha_own)
                                  : quad_bcast<3>(alpha_own);
          }
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i) accm[e][i] *= a4[i];
      } else {
        float alpha[GC];
        if constexpr (GC == 1) {
          alpha[0] = alpha_own;
        } else if constexpr (GC == 8) {  // heads 0..7 sit in the lanes of each 8-lane group
          oct_all(alpha_own, alpha, std::make_integer_sequence<int, 8>{});
        } else {
          alpha[0] = quad_bcast<0>(alpha_own);
          alpha[1] = quad_bcast<1>(alpha_own);
          if constexpr (GC == 4) {
            alpha[2] = quad_bcast<2>(alpha_own);
            alpha[3] = quad_bcast<3>(alpha_own);
          }
        }
#pragma unroll
        for (int h = 0; h < GC; ++h)
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[h][e] *= alpha[h];
      }
      l_own *= alpha_own;
      m_own = m_new;
    }
    const float m_use = (m_own == neg_inf) ? 0.0f : m_own;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(x[r] - m_use);
    l_own += (pr[0] + pr[1]) + (pr[2] + pr[3]);

    if constexpr (PV_MFMA) {
      // A operand (lane 16g + j: score column j, k-slots 8g .. 8g + 7): the probabilities of tokens
      // 4g..4g+3 rounded to the element type, then their residuals.
      u32x4 pa;
      pa[0] = E::pack2(pr[0], pr[1]);
      pa[1] = E::pack2(pr[2], pr[3]);
      pa[2] = E::pack2(pr[0] - E::lo(pa[0]), pr[1] - E::hi(pa[0]));
      pa[3] = E::pack2(pr[2] - E::lo(pa[1]), pr[3] - E::hi(pa[1]));
      // B operand of column block e (lane 16g + j: column j*VEC + e, k-slots 8g .. 8g + 7): element e
      // of this lane's rows 4g..4g+3, twice.  Masked tokens (p = 0) loaded a stand-in row: zero it so
      // 0 * (inf or nan) cannot leak.
#pragma unroll
      for (int w = 0; w < VW; ++w) {
        uint32_t row[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) row[r] = (FULL || ((tile.valid >> r) & 1u)) ? tile.v[r][w] : 0u;
        const uint32_t lo01 = __builtin_amdgcn_perm(row[1], row[0], 0x05040100u);
        const uint32_t lo23 = __builtin_amdgcn_perm(row[3], row[2], 0x05040100u);
        const uint32_t hi01 = __builtin_amdgcn_perm(row[1], row[0], 0x07060302u);
        const uint32_t hi23 = __builtin_amdgcn_perm(row[3], row[2], 0x07060302u);
        accm[2 * w] = E::mfma(pa, u32x4{lo01, lo23, lo01, lo23}, accm[2 * w]);
        accm[2 * w + 1] = E::mfma(pa, u32x4{hi01, hi23, hi01, hi23}, accm[2 * w + 1]);
      }
    } else {
      // PV: token 4g + r, columns j*VEC .. j*VEC + VEC - 1, all heads of the chunk.
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float ph[GC];
        if constexpr (GC == 1) {
          ph[0] = pr[r];
        } else if constexpr (GC == 8) {
          oct_all(pr[r], ph, std::make_integer_sequence<int, 8>{});
        } else {
          ph[0] = quad_bcast<0>(pr[r]);
          ph[1] = quad_bcast<1>(pr[r]);
          if constexpr (GC == 4) {
            ph[2] = quad_bcast<2>(pr[r]);
            ph[3] = quad_bcast<3>(pr[r]);
          }
        }
        // Masked tokens (p = 0) loaded a stand-in row: zero it so 0 * (inf or nan) cannot leak.
        const bool ok = FULL || ((tile.valid >> r) & 1u);
#pragma unroll
        for (int w = 0; w < VW; ++w) {
          const uint32_t word = ok ? tile.v[r][w] : 0u;
          const float v0 = E::lo(word);
          const float v1 = E::hi(word);
#pragma unroll
          for (int h = 0; h < GC; ++h) {
            acc[h][2 * w] = fmaf(ph[h], v0, acc[h][2 * w]);
            acc[h][2 * w + 1] = fmaf(ph[h], v1, acc[h][2 * w + 1]);
          }
        }
      }
    }
  };

  // One tile: wait until `cur` has landed, send out the loads of the tile DEPTH steps ahead (if
  // any), then scores, softmax and PV of `cur` while those loads are in flight.  Slots, the
  // has-next choice and the number of tiles still allowed in flight are compile-time tags, so the
  // register tiles stay in registers and every wait is exact.
  //
  // The wait is explicit.  Loads retire in issue order, so waiting until at most PENDING tiles'
  // worth of operations is outstanding (PENDING = tiles issued after `cur`) is exactly the wait for
  // `cur`'s K DMA and V loads.  The compiler's own counter tracking does not model LDS-DMA completion
  // precisely; with this wait ahead of every use it never has to.  The slot and register tile that
  // the new loads overwrite belong to the tile computed in the previous step, which is finished.
  auto step = [&](const Tile& cur, auto cur_slot, Tile& next, auto next_slot, int next_t0, auto has_next,
                  auto pending) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(wait_vmcnt(decltype(pending)::value * TILE_OPS));
    __asm__ __volatile__("" ::: "memory");
    if constexpr (decltype(has_next)::value) issue_tile(next, decltype(next_slot)::value, next_t0);
    float x[4];
    qk_phase(cur, cur_slot, x);
    if (cur.full)
      pv_phase(cur, x, Flag<true>{});
    else
      pv_phase(cur, x, Flag<false>{});
  };

  // Tiles of this wave: t0 = first + n * step_tokens, n < n_tiles; tile n uses slot n % SLOTS.  The
  // loop is peeled so that every load it issues is unconditional.
  const int step_tokens = kWaves * kTile;
  const int first = p0 + wl * kTile;
  const int n_tiles = first < p_end ? (p_end - first + step_tokens - 1) / step_tokens : 0;
  auto t0_of = [&](int n) { return first + n * step_tokens; };
  constexpr Flag<true> kIssue{};
  Tile tiles[SLOTS];  // tile n lives in tiles[n % SLOTS] and K slot n % SLOTS
  // The first DEPTH tiles go out before the barrier that publishes the staged table (uniform-block
  // path: their block ids were read directly).  All DEPTH are issued even when fewer tiles exist (a
  // missing tile reads masked stand-in rows of the first tile's block and is never computed): an
  // unconditional issue keeps the compiler's view of the memory counter identical on every path
  // into the loop, so it adds no waits of its own, and the explicit waits below only wait longer.
  if constexpr (UB) {
    if (n_tiles > 0) {
      const int pb0 = valid_block(first_raw[0]);
      unroll<DEPTH>([&](auto n) __attribute__((always_inline)) {
        constexpr int N = decltype(n)::value;
        const int t0 = t0_of(N);
        issue_tile_block(tiles[N], N, t0, (N == 0 || t0 <= last) ? valid_block(first_raw[N]) : pb0);
      });
    }
  }
  lds_barrier();
  if constexpr (AP) {
    // The new token's rows into its cache slot (skipped, like the append operator, when its block id
    // is invalid).  Fire and forget: no wave of this launch reads the slot, and the explicit memory
    // waits below stay exact (a store issued before a tile's loads only makes them wait longer).
    if (ap_here && chunk == 0 && wl == 0 && lane < 2 * CPR) {
      const int pb = s_table[(ap_pos >> lb) - blk0];
      if (pb >= 0) {
        uint16_t* dst = (lane < CPR ? p.k_store : p.v_store) + static_cast<int64_t>(pb) * p.block_stride +
                        static_cast<int64_t>(ap_pos & bs_mask) * p.row_stride + static_cast<int64_t>(kvh) * D +
                        (lane % CPR) * 8;
        *reinterpret_cast<u32x4*>(dst) = ap_chunk;
      }
    }
  }
  if constexpr (!UB) {
    if (n_tiles > 0) issue_tile(tiles[0], 0, t0_of(0));
  }

  // Step K of a run of steps that starts at tile n (a multiple of SLOTS): computes tile n + K from
  // slot K % SLOTS and, when ISSUE, first sends out tile n + K + DEPTH into the slot of tile
  // n + K - 1, computed in the step before.  PENDING tiles issued after n + K are still allowed in
  // flight at its wait.
  auto run_step = [&](auto k, int n, auto issue, auto pending) __attribute__((always_inline)) {
    constexpr int K = decltype(k)::value;
    constexpr int CUR = K % SLOTS;
    constexpr int NEXT = (K + DEPTH) % SLOTS;
    step(tiles[CUR], Int<CUR>{}, tiles[NEXT], Int<NEXT>{}, t0_of(n + K + DEPTH), issue, pending);
  };
  if (n_tiles > 0) {
    int n = 0;
    for (; n + SLOTS + DEPTH <= n_tiles; n += SLOTS)
      unroll<SLOTS>([&](auto k) __attribute__((always_inline)) { run_step(k, n, kIssue, Int<DEPTH - 1>{}); });
    // 1 to SLOTS + DEPTH - 1 tiles remain; min(left, DEPTH) of them are in flight.  Step K issues
    // tile n + K + DEPTH if it exists; at its wait, min(DEPTH - 1, left - 1 - K) tiles after n + K
    // have been issued.
    const int left = n_tiles - n;
    unroll<SLOTS + DEPTH - 1>([&](auto l) __attribute__((always_inline)) {
      constexpr int L = decltype(l)::value + 1;
      if (left == L) {
        unroll<L>([&](auto k) __attribute__((always_inline)) {
          constexpr int K = decltype(k)::value;
          constexpr int AHEAD = L - 1 - K < DEPTH - 1 ? L - 1 - K : DEPTH - 1;
          run_step(k, n, Flag<(K + DEPTH < L)>{}, Int<AHEAD>{});
        });
      }
    });
  }

  // Wave totals: sum the four lane groups (they hold disjoint tokens, identical maxima).  The MFMA
  // PV accumulators already hold all of the wave's tokens in every lane group.
  l_own = sum_xor16(l_own);
  l_own = sum_xor32(l_own);
  if constexpr (!PV_MFMA) {
#pragma unroll
    for (int h = 0; h < GC; ++h)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float a = sum_xor16(acc[h][e]);
        acc[h][e] = sum_xor32(a);
      }
  }
  // The staging bytes are reused for the partial accumulators: no DMA may still be writing them
  // and every wave must be done reading its K slots.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  at_epilogue();
  if constexpr (PV_MFMA) {
    // Lane group g holds heads (4g + i) % GC: groups 0 and 1 together every head of an 8-head chunk,
    // group 0 alone every head of a smaller one.
    if (g < (GC == 8 ? 2 : 1)) {
#pragma unroll
      for (int i = 0; i < (GC < 4 ? GC : 4); ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) s_acc[wave][(4 * g + i) % GC][j * VEC + e] = accm[e][i];
    }
  } else if (g == 0) {
#pragma unroll
    for (int h = 0; h < GC; ++h)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s_acc[wave][h][j * VEC + e] = acc[h][e];
  }
  if (g == 0 && j < GC) {
    s_m[wave][j] = m_own;
    s_l[wave][j] = l_own;
  }
  __syncthreads();

  // Merge each KV head's four waves (fixed order) and emit either the final output or a partition
  // record.
  const bool single = (np == 1);
  for (int idx = tid; idx < KVP * heads_here * D; idx += NTHREADS) {
    const int kv = KVP == 1 ? 0 : idx / (heads_here * D);
    const int hd = KVP == 1 ? idx : idx - kv * heads_here * D;
    const int h = hd / D, d = hd % D;
    const int w0 = kv * kWaves;
    float M = neg_inf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w0 + w][h]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = s_m[w0 + w][h];
      const float f = (mw == neg_inf) ? 0.0f : fast_exp2(mw - M);
      L = fmaf(s_l[w0 + w][h], f, L);
      A = fmaf(s_acc[w0 + w][h][d], f, A);
    }
    const int64_t row = static_cast<int64_t>(b) * p.query_heads + (kvh0 + kv) * p.group + chunk * GC + h;
    if (single) {
      p.out[row * D + d] = E::store(A / L);
    } else {
      const int64_t rec = row * p.num_partitions + part;
      store_record(p.ws_acc + rec * D + d, A);
      if (d == 0) {
        store_record(p.ws_ml + rec * 2, M);
        store_record(p.ws_ml + rec * 2 + 1, L);
      }
    }
  }
  if (single || p.counters == nullptr) return;

  // Fused merge.  Every wave waits until its record stores (agent-scope, written through) are
  // acknowledged; after the barrier one thread counts the workgroup's arrival on the (sequence,
  // head slot) counter.  The last of the np arrivals resets the counter for the next call and merges
  // every partition of its heads in partition order, reading the records with agent-scope loads.
  // Nobody waits for anybody, so no workgroup depends on another being scheduled.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);  // keep the record stores above the wait
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    uint32_t* counter = p.counters + static_cast<int64_t>(b) * heads_per_seq + hslot;
    const uint32_t prior = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prior == static_cast<uint32_t>(np - 1);
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1 : 0;
  }
  __syncthreads();
  if (s_last == 0) return;
  for (int r = wave; r < KVP * heads_here; r += NWAVES) {
    const int kv = KVP == 1 ? 0 : r / heads_here;
    const int h = KVP == 1 ? r : r - kv * heads_here;
    const int64_t row = static_cast<int64_t>(b) * p.query_heads + (kvh0 + kv) * p.group + chunk * GC + h;
    merge_partitions<E, D, true>(p, row, np, lane);
  }
}

// Grid schedule: one workgroup per work item, every item of the batch x head slots x partitions
// space, the head slot fastest, then the sequence, then the partition.  Partition-slowest order
// measured 13% faster than partition-fastest on the 128-sequence ragged workload, and it lets the
// early-exiting workgroups of short sequences (partitions past their context) cluster at the end of
// the grid.  The dispatcher places hardware workgroup h on XCD h % 8, so neighbouring head slots
// land on different XCDs.  Keeping all head slots of a (sequence, partition) on one XCD (their rows
// of a token are adjacent in memory) measured 1% slower than this identity order on that workload
// with non-temporal loads, as a read-only probe of the access pattern predicted.
template <class E, int D, int GC, bool QK_MFMA, bool PV_MFMA, bool UB, bool AP>
__global__ __launch_bounds__(kThreads) void pa_partition_kernel(Params p) {
  const int64_t wg = blockIdx.x;
  const int heads_per_seq = p.kv_heads * p.head_chunks;
  const int hslot = static_cast<int>(wg % heads_per_seq);
  const int64_t rest = wg / heads_per_seq;
  const int b = static_cast<int>(rest % p.batch);
  const int part = static_cast<int>(rest / p.batch);
  partition_item<E, D, GC, QK_MFMA, PV_MFMA, UB, AP, 1>(p, static_cast<int>(threadIdx.x), b, hslot, part, p.partition_tokens,
                                            [] {});
}

// Item-map helpers of the work-queue kernel.  kQueueBins counts the key values of its two sorts: a
// sequence's full-partition count (0..256) and the 64-token size class of its partial partition
// (0..128).
constexpr int kQueueBins = 320;
constexpr int kQueueClassTokens = 64;

// Wave 0: s_count[v] <- number of sorted sequences whose key exceeds v, for every bin v.
__device__ __forceinline__ void descending_offsets(int* s_count, int lane) {
  constexpr int PER = kQueueBins / kWave;
  int v[PER];
  int local = 0;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    v[e] = s_count[lane * PER + e];
    local += v[e];
  }
  int suffix = local;  // this lane's bins and every higher lane's
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int other = __shfl_down(suffix, off);
    if (lane + off < kWave) suffix += other;
  }
  int run = suffix - local;
#pragma unroll
  for (int e = PER - 1; e >= 0; --e) {
    s_count[lane * PER + e] = run;
    run += v[e];
  }
}

// Stable counting sort, by descending key, of the sequences whose key(i) is >= 0 (keys below
// kQueueBins) into order[]; every workgroup computes the same order.  before_rounds(s_count) runs
// once the bins hold the descending offsets (s_count[v] = sequences with a larger key).  The
// sequences are placed in rounds of one per thread, in index order: a sequence's position is its
// key's offset, plus the sequences of that key placed in earlier rounds, plus those of lower thread
// index in this round.  O(batch) work per thread for the histogram and at most NT (the workgroup's
// threads) key compares per round, against the O(batch) compares per sequence of a plain rank.
template <int NT, class Key, class Hook>
__device__ __attribute__((always_inline)) inline int queue_sort(int batch, int tid, Key&& key, uint16_t* order,
                                                                int* s_count, int16_t* s_round, Hook&& before_rounds) {
  for (int v = tid; v < kQueueBins; v += NT) s_count[v] = 0;
  __syncthreads();
  for (int i = tid; i < batch; i += NT) {
    const int k = key(i);
    if (k >= 0) atomicAdd(&s_count[k], 1);
  }
  __syncthreads();
  if (tid < kWave) descending_offsets(s_count, tid);
  __syncthreads();
  before_rounds(s_count);
  __syncthreads();
  int placed = 0;
  for (int base = 0; base < batch; base += NT) {
    const int i = base + tid;
    const int k = i < batch ? key(i) : -1;
    s_round[tid] = static_cast<int16_t>(k);
    __syncthreads();
    if (k >= 0) {
      int rank = 0;
      for (int o = 0; o < tid; o += 8) {  // eight keys per 16-byte LDS read
        const u32x4 w = *reinterpret_cast<const u32x4*>(s_round + o);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int other = static_cast<int16_t>(static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1))));
          rank += (o + e < tid && other == k) ? 1 : 0;
        }
      }
      order[s_count[k] + rank] = static_cast<uint16_t>(i);
      ++placed;
    }
    __syncthreads();
    if (k >= 0) atomicAdd(&s_count[k], 1);
    __syncthreads();
  }
  return placed;
}

// Work-queue schedule: as many workgroups as the device holds at once, each running work items
// until none is left.  A grid of one workgroup per item pays a workgroup launch per item (the
// per-workgroup timeline of the 128-sequence ragged workload showed 2-12 us between one
// workgroup's end and the next one's start on the same CU) and a launch plus a context-length load
// for every item past its sequence's context (3672 of its 8192 items, about 4 us each); here only
// items with tokens are scheduled.
//
// Item map, built by every workgroup from the context lengths alone, so all agree on it (P is the
// call's partition size, or the size partition growth picks, also from the contexts alone).  A
// sequence with c > 0 tokens (clamped to the table) has f = c / P full partitions and, when P does
// not divide c, one partial partition of c % P tokens; a context <= 0 has one partial partition of
// no tokens (its item writes the NaN row).  Items are numbered largest first: the full partitions
// level by level (level k: partition k of every sequence with more than k full partitions, the
// sequences by full count, largest first, ties by index), then the partial partitions by size class
// (64-token steps), largest first (ties by index); the head slot is fastest throughout.  The smallest
// items come last, so the workgroups run out of work at nearly the same time.  Both orders are
// stable counting sorts (queue_sort).
//
// Workgroup w runs item w first; every further item comes from the ticket counter
// (gridDim.x + ticket).  Thread 0 claims its workgroup's next ticket at the start of the current
// item's epilogue, decodes it once the epilogue is done and publishes (ticket, sequence, head slot,
// partition) in LDS for the next item.  Claiming at the start of an item instead (one item ahead)
// measured 3% slower on the 128-sequence ragged workload; this order of items measured 1.5%
// faster than partition-major levels over all partitions.  The counter only grows, so every
// workgroup exits after at most items / gridDim.x + 1 tickets.
template <class E, int D, int GC, bool PV_MFMA, bool UB, bool AP, int KVP>
__global__ __launch_bounds__(kThreads * KVP) void pa_partition_queue_kernel(Params p) {
  constexpr int NTHREADS = kThreads * KVP;
  __shared__ uint16_t s_full[kQueueMaxBatch];        // full partitions of sequence b
  __shared__ int16_t s_class[kQueueMaxBatch];        // size class of its partial partition, -1: none
  __shared__ uint16_t s_full_order[kQueueMaxBatch];  // sequences by full count, descending
  __shared__ uint16_t s_part_order[kQueueMaxBatch];  // sequences with a partial, by size class, descending
  __shared__ int s_level[kQueueMaxLevels + 1];       // first item of each full level; [levels] = full items
  __shared__ int s_count[kQueueBins];
  __shared__ __attribute__((aligned(16))) int16_t s_round[NTHREADS];
  __shared__ int s_levels;
  __shared__ int s_partials;
  __shared__ int s_next[2][4];  // ticket, sequence, head slot, partition; by item parity
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int heads_per_seq = (p.kv_heads / KVP) * p.head_chunks;  // work items per (sequence, partition)
  const bool is64 = p.index_is64 != 0;
  const int64_t max_ctx = static_cast<int64_t>(p.max_blocks) << p.bs_log2;
  __shared__ unsigned long long s_tokens;

  // This thread's sequences (tid + r * NTHREADS; the host admits at most kQueueMaxBatch) and their
  // context lengths clamped to the table, loaded once for the partition size and the item map.
  static_assert(kQueueMaxBatch % NTHREADS == 0, "sequences split evenly over the threads");
  constexpr int kSeqPerThread = kQueueMaxBatch / NTHREADS;
  int cc_own[kSeqPerThread];
#pragma unroll
  for (int r = 0; r < kSeqPerThread; ++r) {
    const int i = tid + r * NTHREADS;
    cc_own[r] = 0;
    if (i < p.batch) {
      const int64_t c = index_value(load_raw_index(p.context_lengths, i, is64), is64);
      cc_own[r] = static_cast<int>(c < max_ctx ? c : max_ctx);
    }
  }

  // Partition growth: the largest P << k within the host's limit with (P << k)^2 <= kGrowBalance *
  // W, W = context tokens x head slots per resident workgroup, from the same clamped contexts as the
  // item map, so every workgroup picks the same size.
  int P = p.partition_tokens;
  if (p.grow_max_tokens > P) {
    if (tid == 0) s_tokens = 0;
    __syncthreads();
    unsigned long long own = 0;
#pragma unroll
    for (int r = 0; r < kSeqPerThread; ++r) own += cc_own[r] > 0 ? static_cast<unsigned long long>(cc_own[r]) : 0ull;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) own += __shfl_xor(own, off);
    if (lane == 0) atomicAdd(&s_tokens, own);
    __syncthreads();
    const int64_t tokens = static_cast<int64_t>(s_tokens);  // <= 1024 * 2^31
    const int64_t work = min(tokens * heads_per_seq / static_cast<int64_t>(gridDim.x), int64_t{1} << 40);
    int grow = 0;
    for (int k = 1; k <= kGrowMaxSteps; ++k) {
      const int64_t next = static_cast<int64_t>(P) << k;
      if (next > p.grow_max_tokens || next * next > kGrowBalance * work) break;
      grow = k;
    }
    P = __builtin_amdgcn_readfirstlane(P << grow);
    if (p.grown != nullptr && blockIdx.x == 0 && tid == 0)
      __hip_atomic_store(p.grown, static_cast<uint32_t>(P), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (tid == 0) {
    s_levels = 0;
    s_partials = 0;
  }
#pragma unroll
  for (int r = 0; r < kSeqPerThread; ++r) {
    const int i = tid + r * NTHREADS;
    if (i < p.batch) {
      const int cc = cc_own[r];
      const int rem = cc <= 0 ? 0 : cc % P;
      s_full[i] = static_cast<uint16_t>(cc <= 0 ? 0 : cc / P);
      s_class[i] = static_cast<int16_t>(cc > 0 && rem == 0 ? -1 : (rem + kQueueClassTokens - 1) / kQueueClassTokens);
    }
  }
  __syncthreads();
  // Full order.  Before its rounds the bins hold, for level k, the number of sequences with more than
  // k full partitions: the level's size.
  queue_sort<NTHREADS>(p.batch, tid, [&](int i) { return static_cast<int>(s_full[i]); }, s_full_order, s_count,
                       s_round, [&](const int* count) {
               for (int v = tid; v < kQueueMaxLevels; v += NTHREADS) {
                 s_level[v + 1] = count[v] * heads_per_seq;
                 if (count[v] > 0) atomicMax(&s_levels, v + 1);
               }
             });
  const int levels = __builtin_amdgcn_readfirstlane(s_levels);
  if (tid < kWave) {  // exclusive prefix over the levels: four per lane, then a wave scan
    constexpr int PER = kQueueMaxLevels / kWave;
    int v[PER];
    int local = 0;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int k = lane * PER + e;
      v[e] = k < levels ? s_level[k + 1] : 0;
      local += v[e];
    }
    int incl = local;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int other = __shfl_up(incl, off);
      if (lane >= off) incl += other;
    }
    int run = incl - local;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int k = lane * PER + e;
      run += v[e];
      if (k < levels) s_level[k + 1] = run;
    }
    if (lane == 0) s_level[0] = 0;
  }
  // Partial order (its bins are free again: the full order's rounds are done).
  const int placed = queue_sort<NTHREADS>(p.batch, tid, [&](int i) { return static_cast<int>(s_class[i]); },
                                          s_part_order, s_count, s_round, [](const int*) {});
  if (placed > 0) atomicAdd(&s_partials, placed);
  __syncthreads();
  const int full_items = __builtin_amdgcn_readfirstlane(s_level[levels]);
  const int items = full_items + __builtin_amdgcn_readfirstlane(s_partials) * heads_per_seq;

  // Thread 0: item t -> s_next[slot].
  auto publish = [&](int slot, int t) {
    int b = 0, hslot = 0, part = 0;
    if (t < full_items) {
      int lo = 0, hi = levels - 1;  // the last level starting at or before t
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_level[mid] <= t) lo = mid; else hi = mid - 1;
      }
      const int rem = t - s_level[lo];
      b = s_full_order[rem / heads_per_seq];
      hslot = rem % heads_per_seq;
      part = lo;
    } else if (t < items) {
      const int rem = t - full_items;
      b = s_part_order[rem / heads_per_seq];
      hslot = rem % heads_per_seq;
      part = s_full[b];
    }
    s_next[slot][0] = t;
    s_next[slot][1] = b;
    s_next[slot][2] = hslot;
    s_next[slot][3] = part;
  };
  auto ticket = [&]() -> uint32_t {
    return __hip_atomic_fetch_add(p.queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };

  if (tid == 0) publish(0, blockIdx.x);
  __syncthreads();
  // The item of iteration i is in s_next[i % 2]; thread 0 publishes the next one into the other slot
  // during iteration i (possibly before another wave has read this iteration's slot: an item that
  // ends early returns without a barrier), and the barrier ending iteration i makes it visible.
  for (int slot = 0;; slot ^= 1) {
    const int t = __builtin_amdgcn_readfirstlane(s_next[slot][0]);
    if (t >= items) break;
    const int b = __builtin_amdgcn_readfirstlane(s_next[slot][1]);
    const int hslot = __builtin_amdgcn_readfirstlane(s_next[slot][2]);
    const int part = __builtin_amdgcn_readfirstlane(s_next[slot][3]);
    // Thread 0 only: the next ticket, claimed at the start of the item's epilogue so that the
    // atomic's round trip overlaps the epilogue; its result is first used by publish() below.
    uint32_t claimed = 0;
    bool has_claim = false;
    // The thread index passes through an empty asm statement each item, so nothing computed from it
    // is hoisted out of this loop: per-lane offsets are rebuilt per item instead of holding registers
    // through every item's epilogue (hoisted, they took the 128-dim GQA-4 form to one wave per SIMD).
    int item_tid = tid;
    __asm__ volatile("" : "+v"(item_tid));
    partition_item<E, D, GC, true, PV_MFMA, UB, AP, KVP>(p, item_tid, b, hslot, part, P, [&]() __attribute__((always_inline)) {
      if (tid == 0) {
        claimed = ticket();
        has_claim = true;
      }
    });
    if (tid == 0) {
      if (!has_claim) claimed = ticket();
      publish(slot ^ 1, static_cast<int>(gridDim.x + claimed));
    }
    // Every wave is done with the item's LDS and s_next[slot ^ 1] holds the next item.  An LDS-only
    // barrier: the item's record stores need not be acknowledged before the next item starts (it
    // writes other records).
    lds_barrier();
  }
  // Self-resetting counter: every ticket this workgroup claimed has returned (its value was used), so
  // when the last workgroup counts its exit no claim is outstanding and both words can be zeroed.
  if (p.queue_done != nullptr && tid == 0) {
    const uint32_t done = __hip_atomic_fetch_add(p.queue_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1) {
      __hip_atomic_store(p.queue, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.queue_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Zeroes the work-queue ticket counter in front of a queue launch (a kernel, not a memset, so the
// pair can be captured in a graph).  An agent-scope store, like the tickets' atomics.
__global__ void pa_queue_reset_kernel(uint32_t* queue) {
  if (threadIdx.x == 0) __hip_atomic_store(queue, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------
// Launches.
// Workgroups of one queue-kernel instantiation the current device holds at once (resident
// workgroups per CU, from the kernel's registers and LDS, times the CU count).
struct Residency {
  hipError_t err;
  int per_cu;
};
template <class E, int D, int GC, bool PV_MFMA, bool UB, bool AP, int KVP>
hipError_t queue_capacity(int64_t* capacity) {
  static const Residency r = [] {
    Residency out{hipSuccess, 0};
    out.err = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &out.per_cu, reinterpret_cast<const void*>(&pa_partition_queue_kernel<E, D, GC, PV_MFMA, UB, AP, KVP>),
        kThreads * KVP, 0);
    return out;
  }();
  if (r.err != hipSuccess) return r.err;
  constexpr int kMaxDevices = 256;
  static std::atomic<int> cus[kMaxDevices];
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  int n = device >= 0 && device < kMaxDevices ? cus[device].load(std::memory_order_relaxed) : 0;
  if (n == 0) {
    err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
    if (err != hipSuccess) return err;
    if (device >= 0 && device < kMaxDevices) cus[device].store(n, std::memory_order_relaxed);
  }
  *capacity = static_cast<int64_t>(r.per_cu > 0 ? r.per_cu : 1) * n;
  return hipSuccess;
}

// KV-head pairs.  The work queue can run two KV heads per workgroup (8 waves, four per KV head).  At
// head_dim 128 a token's row of one KV head is 256 bytes and the two heads' rows are adjacent; the
// workgroup's two wave groups read them at nearly the same time.  A read-only probe of the
// 128-sequence ragged access pattern streamed 7.0 TB/s that way against 6.5 TB/s with one head per
// workgroup, at equal workgroups, bytes and loads in flight.  Every KV head runs exactly as in a
// one-head workgroup, so the outputs do not change.
//
// The pairs hold a CU's one 8-wave workgroup in step: an item's prologue and epilogue no longer
// overlap another workgroup's streaming on the same CU, and the CU's share of the call's tail is
// coarser.  They pay on long calls of long items and lose on short ones, so they run only with head
// chunks of at most 4 (8-head chunks measured 0.5-8% slower), without partition growth, with
// partitions of at least kPairMinPartitionTokens and at least kPairMinRows (sequence, KV head)
// rows.  Measured against one head per workgroup (head_dim 128, fused): 128 sequences of 1k-16k
// tokens, GQA 32x8, P 8192 -2.0% and P 4096 -1.7%; 32 sequences at P 4096 +4.5%; 64 sequences
// with growth +2.1%; 512 sequences with growth -0.9%.
template <int D, int GC, bool PV_MFMA, bool UB>
constexpr bool kPairsKvHeads = D == 128 && GC <= 4 && PV_MFMA && UB;
constexpr int kPairMinPartitionTokens = 4096;
constexpr int64_t kPairMinRows = 1024;
__device__ __host__ constexpr bool pair_kv_heads(int kv_heads, int batch, int partition_tokens, int grow_max_tokens) {
  return kv_heads % 2 == 0 && grow_max_tokens <= partition_tokens && partition_tokens >= kPairMinPartitionTokens &&
         static_cast<int64_t>(batch) * kv_heads >= kPairMinRows;
}

template <class E, int D, int GC, bool PV_MFMA, bool UB, bool AP, int KVP>
hipError_t launch_queue_kernel(const Params& prm, int64_t items, hipStream_t stream) {
  int64_t capacity = 0;
  const hipError_t err = queue_capacity<E, D, GC, PV_MFMA, UB, AP, KVP>(&capacity);
  if (err != hipSuccess) return err;
  const int64_t own = items / KVP;  // this kernel's work items (KVP KV heads each)
  const int64_t grid = own < capacity ? own : capacity;
  hipLaunchKernelGGL((pa_partition_queue_kernel<E, D, GC, PV_MFMA, UB, AP, KVP>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kThreads * KVP), 0, stream, prm);
  return hipGetLastError();
}

// The partition launch for `items` work items (one KV head each).  For a queue-eligible call (a
// split-K shape whose item map fits the queue kernel; prm.queue is then its ticket counter) the
// work-queue schedule runs when asked for, or, by default, when the items exceed what the device
// holds at once of the one-head queue kernel and partitions hold at least kQueueMinPartitionTokens
// tokens; otherwise one workgroup per item.  With `chosen`, nothing is launched: the schedule is
// stored there instead.
template <class E, int D, int GC, bool QK_MFMA, bool PV_MFMA, bool UB, bool AP>
hipError_t launch_partition_kernel(const Params& prm, int64_t items, int schedule, bool queue_ok, hipStream_t stream,
                                   int* chosen) {
  if constexpr (QK_MFMA) {
    if (queue_ok) {
      int64_t capacity = 0;
      const hipError_t err = queue_capacity<E, D, GC, PV_MFMA, UB, AP, 1>(&capacity);
      if (err != hipSuccess) return err;
      if (schedule == kScheduleQueue ||
          (schedule == kScheduleAuto && items > capacity && prm.partition_tokens >= kQueueMinPartitionTokens)) {
        if (chosen != nullptr) {
          *chosen = RK_PA_SCHEDULE_QUEUE;
          return hipSuccess;
        }
        if (prm.queue_done == nullptr)
          hipLaunchKernelGGL(pa_queue_reset_kernel, dim3(1), dim3(kWave), 0, stream, prm.queue);
        if constexpr (kPairsKvHeads<D, GC, PV_MFMA, UB>) {
          if (pair_kv_heads(prm.kv_heads, prm.batch, prm.partition_tokens, prm.grow_max_tokens))
            return launch_queue_kernel<E, D, GC, PV_MFMA, UB, AP, 2>(prm, items, stream);
        }
        return launch_queue_kernel<E, D, GC, PV_MFMA, UB, AP, 1>(prm, items, stream);
      }
    }
  }
  if (chosen != nullptr) {
    *chosen = RK_PA_SCHEDULE_GRID;
    return hipSuccess;
  }
  hipLaunchKernelGGL((pa_partition_kernel<E, D, GC, QK_MFMA, PV_MFMA, UB, AP>), dim3(static_cast<uint32_t>(items)),
                     dim3(kThreads), 0, stream, prm);
  return hipGetLastError();
}

template <class E, int D, int GC, bool QK_MFMA, bool PV_MFMA, bool AP>
hipError_t launch_partition_ub(const Params& prm, const Launch& l) {
  if (prm.bs_log2 >= 4)
    return launch_partition_kernel<E, D, GC, QK_MFMA, PV_MFMA, true, AP>(prm, l.items, l.schedule, l.queue_ok,
                                                                         l.stream, l.chosen);
  return launch_partition_kernel<E, D, GC, QK_MFMA, PV_MFMA, false, AP>(prm, l.items, l.schedule, l.queue_ok, l.stream,
                                                                        l.chosen);
}

template <class E, int D, int GC>
hipError_t launch_partition(const Params& prm, int variant, const Launch& l) {
  const bool pv_mfma = variant == RK_PA_VARIANT_MFMA;
  if constexpr (D == 256 && GC == 8) {
    // Built with PV on MFMA only: with PV on fp32 FMAs the 8-head accumulators spill at head_dim 256,
    // and the host gives those variants chunks of 4.
    if (!pv_mfma) return hipErrorInvalidValue;
    if (prm.new_k != nullptr) return launch_partition_ub<E, D, GC, true, true, true>(prm, l);
    return launch_partition_ub<E, D, GC, true, true, false>(prm, l);
  } else {
    if (prm.new_k != nullptr)  // validated: an MFMA variant
      return pv_mfma ? launch_partition_ub<E, D, GC, true, true, true>(prm, l)
                     : launch_partition_ub<E, D, GC, true, false, true>(prm, l);
    if (pv_mfma) return launch_partition_ub<E, D, GC, true, true, false>(prm, l);
    if (variant == RK_PA_VARIANT_MFMA_QK) return launch_partition_ub<E, D, GC, true, false, false>(prm, l);
    return launch_partition_ub<E, D, GC, false, false, false>(prm, l);
  }
}

template <class E, int D>
hipError_t launch_all(const Params& prm, int gc, int variant, const Launch& l, bool partitions, bool reduce) {
  hipError_t err = hipSuccess;
  if (partitions) {
    if (gc == 1)
      err = launch_partition<E, D, 1>(prm, variant, l);
    else if (gc == 2)
      err = launch_partition<E, D, 2>(prm, variant, l);
    else if (gc == 4)
      err = launch_partition<E, D, 4>(prm, variant, l);
    else
      err = launch_partition<E, D, 8>(prm, variant, l);
  }
  if (err != hipSuccess || !reduce || l.chosen != nullptr) return err;
  const hipStream_t stream = l.stream;
  const int64_t rows = static_cast<int64_t>(prm.batch) * prm.query_heads;
  const int64_t rgrid = (rows + kWaves - 1) / kWaves;
  hipLaunchKernelGGL((pa_reduce_kernel<E, D>), dim3(static_cast<uint32_t>(rgrid)), dim3(kThreads),
                     0, stream, prm);
  return hipGetLastError();
}

using bf16 = Bf16;
using fp16 = Fp16;

}  // namespace

#define RK_PA_UNIT_DEFINE(ELEMENT, HEAD_DIM)                                               \
  RK_PA_UNIT_LAUNCHER(ELEMENT, HEAD_DIM) {                                                \
    return launch_all<ELEMENT, HEAD_DIM>(prm, gc, variant, l, partitions, reduce);        \
  }
#define RK_PA_UNIT_EXPAND(ELEMENT, HEAD_DIM) RK_PA_UNIT_DEFINE(ELEMENT, HEAD_DIM)
RK_PA_UNIT_EXPAND(RK_PA_UNIT_ELEMENT, RK_PA_UNIT_HEAD_DIM)

}  // namespace rk_pa
