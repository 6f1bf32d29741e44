// Shared gfx950 device helpers for the VMonarch kernels.
//
// Register layouts used throughout (v_mfma_f32_32x32x16_{bf16,f16}, wave64, l = lane):
//   A (32 x 16): lane l holds A[l % 32][8 * (l / 32) + e], e = 0..7
//   B (16 x 32): lane l holds B[8 * (l / 32) + e][l % 32]
//   C (32 x 32): lane l holds C[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32], r = 0..15
// ds_read_tr16_b64: within each 16-lane group, lane i supplies the address of 4 consecutive
// 16-bit elements; lanes 4t..4t+3 together cover row t (16 elements).  Lane i receives
// element i of rows 0..3, i.e. a column of the 4 x 16 block.
// Both were confirmed on an MI355X by a probe of the builtins' lane layouts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace vmo {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

#define VMO_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element-type traits: storage type, 8-wide MFMA operand vector and the MFMA itself.
template <bool F16> struct Elem;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <> struct Elem<false> {
  using T = __bf16;
  using V8 = bf16x8;
  using V4 = bf16x4;
  using V2 = bf16x2;
  __device__ static inline f32x16 mfma(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // round two floats to a packed pair (v_cvt_pk_bf16_f32, round to nearest even)
  __device__ static inline V2 pack2(float a, float b) { return V2{(T)a, (T)b}; }
};
template <> struct Elem<true> {
  using T = _Float16;
  using V8 = f16x8;
  using V4 = f16x4;
  using V2 = f16x2;
  __device__ static inline f32x16 mfma(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline V2 pack2(float a, float b) { return V2{(T)a, (T)b}; }
};

// 16-byte chunk swizzle of LDS tiles whose rows are >= 8 chunks wide: chunk c of row r is
// stored at chunk c ^ swz(r).  Eight consecutive rows map one logical chunk to eight distinct
// bank groups (row-wise ds_read_b128 of an MFMA A operand), and a 4-row x 2-chunk block (one
// 16-lane group of ds_read_tr16_b64) also lands on eight distinct bank groups.
__device__ __forceinline__ int swz(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }

// Bank-conflict-free chunk swizzle for gfx950's 64-bank LDS (256 bytes per cycle), for tiles with
// RB-byte rows (RB = 64, 128, 256 or 512): chunk c of row r is stored at chunk c ^ swz_rows<RB>(r).
//  * ds_read_b128 of 16 consecutive rows at one logical chunk (an MFMA A operand, 16 lanes per
//    cycle) hits 16 distinct 16-byte bank groups: for RB >= 256 the map r -> f(r) is a bijection
//    on r mod 16; for RB = 128 (two rows per bank line) it is a bijection on each row parity.
//  * ds_read_tr16_b64 of 4 aligned rows x 4 aligned chunks (32 lanes per cycle) hits 16 distinct
//    groups: f(r) >> 2 differs between the rows that share a bank line position.
//  * RB = 64 (four rows per bank line, four chunks per row): f(r) = (r / 4) % 4, so 16 consecutive rows at
//    one logical chunk take the 16 (row % 4, chunk) positions of a bank line.
// f(r + 8) = f(r) ^ 2 and f(r + 16) = f(r).
template <int RB>
__device__ __forceinline__ int swz_rows(int r) {
  static_assert(RB == 64 || RB == 128 || RB == 256 || RB == 512, "row width");
  if constexpr (RB == 64) return (r >> 2) & 3;
  else if constexpr (RB == 128) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return ((r & 3) << 2) | ((r >> 2) & 3);
}

// XCD-aware block order for a grid of nblocks (a multiple of 8): block b runs on XCD b % 8, so give
// each XCD a contiguous run of logical blocks (neighbouring tiles / rows then share that XCD's L2).
__device__ __forceinline__ int xcd_remap(int nblocks) {
  const int per_xcd = nblocks >> 3;
  return (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
}

__device__ __forceinline__ float wave_max32(float x) {
  // combine lane l with lane l ^ 32
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// 16-byte global -> LDS copy without a register round trip.  The LDS destination of lane l is
// lds_wave_base + 16 * l (lds_wave_base must be wave-uniform).
__device__ __forceinline__ void g2l_16(const void* g, VMO_LDS void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, lds_wave_base, 16, 0, 0);
}

// The same copy issued from inline asm, for pipelines that order their LDS traffic themselves.
// The compiler cannot see this store to LDS, so it adds no wait of its own before later LDS reads
// (with the builtin, every ds_read_tr16_b64 -- whose memory operand has no alias information --
// waits for the most recent copy, which serialises a prefetch with the reads of the current
// tile).  The caller must order the copy with tile_sync<>() below.  lds_wave_base is an LDS byte
// address; it goes through M0, which the asm names as clobbered.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_async(const void* g, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_wave_base))
               : "m0");
}
// 4-byte variant of dma16_async: lane l copies one dword to lds_wave_base + 4 * l.
__device__ __forceinline__ void dma4_async(const void* g, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_wave_base))
               : "m0");
}
// A wave-uniform 64-bit value, moved to scalar registers (the compiler may otherwise keep a
// uniform pointer in VGPRs and do its address arithmetic on the vector unit).
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
         (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
}

// As dma16_async, with the source split into a wave-uniform 64-bit base (an SGPR pair) and a
// per-lane 32-bit byte offset: a copy costs no vector instructions when the offsets are reused.
__device__ __forceinline__ void dma16_async_s(uint64_t sbase, uint32_t voff, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(uniform64(sbase)), "s"(__builtin_amdgcn_readfirstlane(lds_wave_base))
               : "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier for a dma16_async pipeline: this wave's own copies except the newest
// `PENDING` have landed, its LDS reads have returned, then all waves meet.  After it, every copy
// older than the newest PENDING of each wave is visible to all waves.  The memory clobber keeps
// LDS accesses on their side of the barrier.
template <int PENDING>
__device__ __forceinline__ void tile_sync() {
  static_assert(PENDING >= 0 && PENDING < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(PENDING) : "memory");
}

template <class V8>
__device__ __forceinline__ V8 lds_read8(const VMO_LDS char* p) {
  return *reinterpret_cast<const VMO_LDS V8*>(p);
}

// Two transposed 4-element reads concatenated into one 8-element MFMA operand.
template <class V8>
__device__ __forceinline__ V8 lds_read_tr8(const VMO_LDS char* p0, const VMO_LDS char* p1) {
  i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VMO_LDS i16x4*)p0);
  i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((VMO_LDS i16x4*)p1);
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  i16x8 c = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(V8, c);
}

template <class T>
__device__ __forceinline__ T to_elem(float x) { return static_cast<T>(x); }

// How a result row is written: in the inputs' 16-bit type, into an fp32 buffer (added to or
// overwritten), or in the 16-bit type as the sum with an fp32 base row (the last of several
// contributions to one gradient).
enum { kGradStore = 0, kGradAddF32 = 1, kGradStoreF32 = 2, kGradSumStore = 3 };
__device__ __forceinline__ int grad_mode(int flags, int accum_bit, int f32_bit, int sum_bit = 0) {
  return (flags & sum_bit) ? kGradSumStore
         : (flags & accum_bit) ? kGradAddF32 : (flags & f32_bit) ? kGradStoreF32 : kGradStore;
}

// Width of a 16-bit tile row in LDS for a head dim w: a 16-wide head (q / k, a value tensor, dO) is laid out 32
// wide with each row's two 16-byte chunks stored twice, so that the 32-wide operand reads apply unchanged:
// products over the head dim take one 16-dim MFMA step, and products that output it (P.V, dQ, dK, dV, u, z)
// fill accumulator rows 16-31 with a copy of rows 0-15, which are not stored (CW = 16 below).
constexpr int tile_w(int w) { return w < 32 ? 32 : w; }

// Write a wave's 32-row result tile -- acc[a][r] is the value at (row l32, column 32 a + 8 (r / 4) +
// 4 hl + r % 4), the transposed accumulator layout every kernel here ends with -- through a 4 KB LDS
// patch, so that 8 consecutive lanes write one row's 128-byte segment (32 fp32 or 64 16-bit columns)
// instead of every lane writing 8- or 16-byte pieces of 32 rows (rows are often far apart: tokens of
// one grid column, or rows of a strided layout).  Only rows rbegin .. nrows-1 are written; f may differ
// per lane (it scales the lane's own row l32).  One wave writes and reads its own patch (LDS accesses
// of a wave complete in order); the caller makes sure no other wave still uses that LDS.  Used by the
// flash-entropy forward (o) and backward (gradients) and both L-step kernels (u / z, gradients).
// kEpiPatchBytes is the 32-row patch.  CW = 16: each accumulator block holds 16 valid columns (rows 0-15 of the transposed accumulator; the 16-wide
// heads, whose LDS tiles hold every row twice), stored as columns 16 a .. 16 a + 15.  PROWS = 16: a 2 KB patch
// that takes the 32 rows in two halves (for kernels whose LDS budget is that tight).
constexpr int kEpiPatchBytes = 32 * 32 * 4;
template <bool F16, int CW = 32, int PROWS = 32>
__device__ __forceinline__ void store_acc_rows(VMO_LDS float* patch, const f32x16* acc, int nacc, float f, int mode,
                                               char* row0, int64_t row_stride_bytes, int nrows, int lane,
                                               int rbegin = 0, const char* src0 = nullptr,
                                               int64_t src_stride_bytes = 0) {
  using T = typename Elem<F16>::T;
  using V4 = typename Elem<F16>::V4;
  using V8 = typename Elem<F16>::V8;
  const int hl = lane >> 5, l32 = lane & 31, rr0 = lane >> 3, c = lane & 7;
  static_assert(CW == 16 || CW == 32, "block width");
  static_assert(PROWS == 16 || PROWS == 32, "patch rows");
  if (CW == 32 && PROWS == 32 && mode == kGradStore && nacc % 2 == 0) {
    // 16-bit rows: two blocks (64 columns) per pass, so that 8 lanes write a whole 128-byte segment
    VMO_LDS char* pb = (VMO_LDS char*)patch;   // [32 rows][8 chunks of 16 bytes], chunk ^ (row & 7)
    for (int a = 0; a < nacc; a += 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {   // columns 32 h + 8 j + 4 hl .. +3: chunk 4 h + j, half hl
          V4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = to_elem<T>(acc[a + h][4 * j + e] * f);
          *(VMO_LDS V4*)(pb + l32 * 128 + ((4 * h + j) ^ (l32 & 7)) * 16 + hl * 8) = x;
        }
#pragma unroll
      for (int i = 0; i < 4; ++i) {   // rows rr0 + 8 i, chunk c (columns 8 c .. 8 c + 7)
        const int rr = rr0 + 8 * i;
        const V8 x = *(const VMO_LDS V8*)(pb + rr * 128 + (c ^ (rr & 7)) * 16);
        if (rr >= rbegin && rr < nrows) *(V8*)(row0 + rr * row_stride_bytes + (int64_t)(32 * a + 8 * c) * 2) = x;
      }
    }
    return;
  }
  const int esize = mode == kGradStore || mode == kGradSumStore ? 2 : 4;
  for (int a = 0; a < nacc; ++a)
#pragma unroll
  for (int h = 0; h < 32 / PROWS; ++h) {   // rows h PROWS .. h PROWS + PROWS - 1 through the patch
    if (PROWS == 32 || (l32 / PROWS) == h) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {   // row l32, 16-byte chunk 2 j + hl, swizzled by row against bank conflicts
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[a][4 * j + e] * f;
        *(VMO_LDS f32x4*)(patch + (l32 % PROWS) * 32 + ((2 * j + hl) ^ (l32 & 7)) * 4) = v;
      }
    }
    // The lanes read rows other lanes wrote: to the compiler's one-thread view, a lane that wrote nothing in this
    // half re-reads the address it read in the last one, and it forwarded that old value (the reads of a wave
    // follow its writes in order in the hardware; this keeps the compiler from caching across the exchange).
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < PROWS / 8; ++i) {   // rows rr0 + 8 i of the patch, chunk c: 8 lanes per row
      const int pr = rr0 + 8 * i, rr = h * PROWS + pr;
      const f32x4 v = *(const VMO_LDS f32x4*)(patch + pr * 32 + (c ^ (pr & 7)) * 4);
      if (rr >= rbegin && rr < nrows && 4 * c < CW) {
        char* dst = row0 + rr * row_stride_bytes + (int64_t)(CW * a + 4 * c) * esize;
        if (mode == kGradStore || mode == kGradSumStore) {
          // (sum: the base row src0 is fp32, same columns; the product came through LDS, so the
          // sum is its own rounding, as adding the fp32 store of this result would be)
          const f32x4 b = mode == kGradSumStore
                              ? *(const f32x4*)(src0 + rr * src_stride_bytes + (int64_t)(CW * a + 4 * c) * 4)
                              : f32x4{0.f, 0.f, 0.f, 0.f};
          V4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = to_elem<T>(mode == kGradSumStore ? b[e] + v[e] : v[e]);
          *(V4*)dst = x;
        } else {
          f32x4* ptr = (f32x4*)dst;
          *ptr = mode == kGradAddF32 ? *ptr + v : v;
        }
      }
    }
    asm volatile("" ::: "memory");   // this half's reads before the next half's (or block's) writes
  }
}

// Runs step(i, operand(i)) for i = 0 .. N-1 with operand(i + PF) read before step(i), so that the
// LDS reads of the next PF products are in flight behind each MFMA (at one or two waves per SIMD no
// other wave hides a read's latency, and the scheduler otherwise issues each read just before its
// product).  operand(i) and step(i, .) must be inlinable with compile-time i after unrolling.
// PF = 0 reads each operand just before its product (the scheduler's choice).
template <int N, int PF, class Operand, class Step>
__device__ __forceinline__ void prefetched_chain(Operand operand, Step step) {
  static_assert(N >= 1 && PF >= 0, "chain");
  if constexpr (PF == 0) {
#pragma unroll
    for (int i = 0; i < N; ++i) step(i, operand(i));
  } else {
    using V = decltype(operand(0));
    V ring[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i)
      if (i < N) ring[i] = operand(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const V cur = ring[i % PF];
      if (i + PF < N) ring[i % PF] = operand(i + PF);
      step(i, cur);
    }
  }
}

// Compile-time loop: f(std::integral_constant<int, I>{}) for I = B .. E - 1.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Pins the order of an unrolled operand chain (prefetched_chain) for the scheduler: step i has
// Chain::reads(i) LDS reads and Chain::mfmas(i) MFMAs, and its reads are issued Chain::ahead(i) steps
// before its MFMAs, i.e. after the MFMAs of step i - ahead(i); Chain::lead() more LDS reads (issued before
// the chain in the same region) go first.  Without it the scheduler moves each read next to its MFMA
// under register pressure and waits for it there.  Place it after the chain's code.
template <class Chain, int N>
__device__ __forceinline__ void pin_chain() {
  constexpr auto reads_after = [](int i) {   // LDS reads issued after the MFMAs of step i (i = -1: first)
    int n = i == -1 ? Chain::lead() : 0;
    for (int j = 0; j < N; ++j) {
      const int at = j - Chain::ahead(j);
      if (at == i || (i == -1 && at < 0)) n += Chain::reads(j);
    }
    return n;
  };
  if constexpr (reads_after(-1) > 0) __builtin_amdgcn_sched_group_barrier(0x100, reads_after(-1), 0);
  static_for<0, N>([&](auto ic) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value;
    __builtin_amdgcn_sched_group_barrier(0x008, Chain::mfmas(i), 0);
    if constexpr (reads_after(i) > 0) __builtin_amdgcn_sched_group_barrier(0x100, reads_after(i), 0);
  });
}

}  // namespace vmo
