// MI355X (gfx950) kernels and C ABI of the LTHC read / write / materialise
// interface.  Declarations and the reference interface each entry point
// replaces are in include/lthc.h.
//
// Layout.  High-resolution activations are NHWC [B, H, H, C] with H = G*4;
// the 16 taps of cell m = (gy, gx) are the 4x4 patch h = 4gy + sy,
// w = 4gx + sx, so each tap row of a cell is one contiguous run of 4*C
// elements and consecutive cells along gx continue that run.  Workspace
// tensors are [B, G*G, C].  Weights are [C, 16] (tap index fastest).
//
// Every kernel here is HBM-bandwidth bound: 1 to 24 fp32 FMAs per element
// moved.  Lanes of a wavefront run along the channel axis, so one wavefront
// load covers a contiguous 512 B .. 1 KiB run of one tap.  The per-channel
// weights a thread needs are loaded into VGPRs once per block and reused for
// every cell the block visits.  Each cell iteration is written as two phases
// separated by a scheduling barrier: (1) issue every vector load of the cell,
// (2) widen, FMA, narrow and store.  Loads are never placed under a
// data-dependent branch (padding layers read a valid clamped pointer and are
// masked by a select), so a wavefront keeps all of a cell's loads in flight
// instead of waiting on each one.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <initializer_list>
#include <numeric>
#include <string>
#include <type_traits>
#include <utility>

#include "../../include/lthc.h"

#define LTHC_DEV __device__ __forceinline__

namespace {

constexpr int kS = 4;        // cell side
constexpr int kK = kS * kS;  // taps per cell
constexpr int kBlock = 256;  // threads per block of the cell kernels

// ---------------------------------------------------------------------------
// Element formats
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int DT>
struct Fmt {
  static constexpr int bytes = DT == LTHC_F32 ? 4 : 2;
};

template <int DT>
LTHC_DEV float widen1(uint32_t h16) {
  if constexpr (DT == LTHC_BF16) return __uint_as_float(h16 << 16);
  else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h16)));
}

template <int DT>
LTHC_DEV void unpack2(uint32_t w, float& a, float& b) {
  if constexpr (DT == LTHC_BF16) {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  } else {
    const f16x2_t h = __builtin_bit_cast(f16x2_t, w);
    a = static_cast<float>(h.x);
    b = static_cast<float>(h.y);
  }
}

// Round-to-nearest-even narrowing (v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
template <int DT>
LTHC_DEV uint32_t pack2(float a, float b) {
  if constexpr (DT == LTHC_BF16) {
    const bf16x2_t r = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, r);
  } else {
    const f16x2_t r = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
    return __builtin_bit_cast(uint32_t, r);
  }
}

// Narrowing of one value to a 16-bit format (round to nearest even), bits in the low half.
template <int DT>
LTHC_DEV uint32_t narrow1(float v) {
  if constexpr (DT == LTHC_BF16) return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// Raw storage of N consecutive elements of format DT: whole dwords, or one
// 16-bit element (kBytes == 2, held in the low half of w[0]).
template <int DT, int N>
struct Raw {
  static constexpr int kBytes = N * Fmt<DT>::bytes;
  static constexpr int kWords = kBytes >= 4 ? kBytes / 4 : 1;
  static_assert(kBytes == 2 || kWords <= 2 || kWords % 4 == 0, "raw vector width");
  uint32_t w[kWords];
};

// One vector load (dwordx1/x2/x4, several x4 for wider runs) of the raw
// bytes at base + boff; NT = streaming (non-temporal).  With a uniform base
// and a 32-bit offset (Off = uint32_t) this is the saddr + voffset form, so
// the per-lane address costs one VGPR and no 64-bit arithmetic.
template <int DT, int N, bool NT = false, typename Off = int64_t>
LTHC_DEV void load_at(const void* __restrict__ base, Off boff, Raw<DT, N>& r) {
  constexpr int W = Raw<DT, N>::kWords;
  const char* q = static_cast<const char*>(base) + boff;
  if constexpr (Raw<DT, N>::kBytes == 2) {
    r.w[0] = NT ? __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(q)) : *reinterpret_cast<const uint16_t*>(q);
  } else if constexpr (W == 1) {
    r.w[0] = NT ? __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(q)) : *reinterpret_cast<const uint32_t*>(q);
  } else if constexpr (W == 2) {
    const u32x2_t t = NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(q)) : *reinterpret_cast<const u32x2_t*>(q);
    r.w[0] = t.x;
    r.w[1] = t.y;
  } else {
#pragma unroll
    for (int j = 0; j < W / 4; ++j) {
      const u32x4_t* v = reinterpret_cast<const u32x4_t*>(q) + j;
      const u32x4_t t = NT ? __builtin_nontemporal_load(v) : *v;
      r.w[4 * j + 0] = t.x;
      r.w[4 * j + 1] = t.y;
      r.w[4 * j + 2] = t.z;
      r.w[4 * j + 3] = t.w;
    }
  }
}

// Element-index form.
template <int DT, int N, bool NT = false>
LTHC_DEV void load_raw(const void* __restrict__ p, int64_t i, Raw<DT, N>& r) {
  load_at<DT, N, NT>(p, i * Fmt<DT>::bytes, r);
}

template <int DT, int N>
LTHC_DEV void unpack_raw(const Raw<DT, N>& r, float (&v)[N]) {
  if constexpr (DT == LTHC_F32) {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = __uint_as_float(r.w[j]);
  } else if constexpr (N == 1) {
    v[0] = widen1<DT>(r.w[0]);
  } else {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) unpack2<DT>(r.w[j], v[2 * j], v[2 * j + 1]);
  }
}

template <int DT, int N>
LTHC_DEV void load_vec(const void* __restrict__ p, int64_t i, float (&v)[N]) {
  Raw<DT, N> r;
  load_raw<DT, N>(p, i, r);
  unpack_raw<DT, N>(r, v);
}

template <int DT, int N, bool NT = false, typename Off = int64_t>
LTHC_DEV void store_at(void* __restrict__ base, Off boff, const float (&v)[N]) {
  char* q = static_cast<char*>(base) + boff;
  if constexpr (N * Fmt<DT>::bytes == 2) {
    const uint16_t h = static_cast<uint16_t>(narrow1<DT>(v[0]));
    if (NT) __builtin_nontemporal_store(h, reinterpret_cast<uint16_t*>(q));
    else *reinterpret_cast<uint16_t*>(q) = h;
  } else {
    constexpr int W = N * Fmt<DT>::bytes / 4;
    uint32_t w[W];
    if constexpr (DT == LTHC_F32) {
#pragma unroll
      for (int j = 0; j < N; ++j) w[j] = __float_as_uint(v[j]);
    } else {
#pragma unroll
      for (int j = 0; j < N / 2; ++j) w[j] = pack2<DT>(v[2 * j], v[2 * j + 1]);
    }
    if constexpr (W == 1) {
      if (NT) __builtin_nontemporal_store(w[0], reinterpret_cast<uint32_t*>(q));
      else *reinterpret_cast<uint32_t*>(q) = w[0];
    } else if constexpr (W == 2) {
      const u32x2_t t = {w[0], w[1]};
      if (NT) __builtin_nontemporal_store(t, reinterpret_cast<u32x2_t*>(q));
      else *reinterpret_cast<u32x2_t*>(q) = t;
    } else {
      static_assert(W % 4 == 0, "store width");
#pragma unroll
      for (int j = 0; j < W / 4; ++j) {
        const u32x4_t t = {w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
        if (NT) __builtin_nontemporal_store(t, reinterpret_cast<u32x4_t*>(q) + j);
        else reinterpret_cast<u32x4_t*>(q)[j] = t;
      }
    }
  }
}

template <int DT, int N, bool NT = false>
LTHC_DEV void store_vec(void* __restrict__ p, int64_t i, const float (&v)[N]) {
  store_at<DT, N, NT>(p, i * Fmt<DT>::bytes, v);
}

// N consecutive weights of format WDT, widened to fp32 (one vector load
// where the width allows it).
template <int WDT, int N>
LTHC_DEV void load_wvec(const void* __restrict__ p, int64_t i, float (&v)[N]) {
  if constexpr (WDT == LTHC_F32 || N % 2 == 0) {
    load_vec<WDT, N>(p, i, v);
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = widen1<WDT>(static_cast<const uint16_t*>(p)[i + j]);
  }
}

// Scalar weight of a runtime dtype (small kernels only).
LTHC_DEV float load_w(const void* __restrict__ p, int dt, int64_t i) {
  if (dt == LTHC_F32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  if (dt == LTHC_BF16) return widen1<LTHC_BF16>(h);
  return widen1<LTHC_F16>(h);
}

// Round one value to format DT (round to nearest even; identity for fp32).
template <int DT>
LTHC_DEV float round_w(float v) {
  if constexpr (DT == LTHC_F32) return v;
  else if constexpr (DT == LTHC_BF16) return static_cast<float>(static_cast<__bf16>(v));
  else return static_cast<float>(static_cast<_Float16>(v));
}

// fp16 outputs of an fma chain are rounded once from the fp32 result: the empty asm keeps the compiler from folding
// the last fma and the narrowing into a mixed-precision fma (one rounding of the exact value) for some lanes or
// kernels and not others, so every kernel producing the same quantity gives the same bits.
template <int DT, int N>
LTHC_DEV void hold_f32(float (&v)[N]) {
  if constexpr (DT == LTHC_F16) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
  }
}

LTHC_DEV void store_w(void* __restrict__ p, int dt, int64_t i, float v) {
  if (dt == LTHC_F32) {
    static_cast<float*>(p)[i] = v;
  } else if (dt == LTHC_BF16) {
    static_cast<__bf16*>(p)[i] = static_cast<__bf16>(v);
  } else {
    static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  }
}

struct PtrPack {
  const void* p[LTHC_MAX_LAYERS];
};

// Walks consecutive cells without divisions.  hoff = element offset of tap
// (0, 0), channel 0 of the current cell in the NHWC tensor; zoff = cell * C.
// Stepping to the next cell adds 4C to hoff, plus 3 high-res rows (3HC) when
// the cell row wraps (the next cell row starts 4 high-res rows down; the
// batch boundary needs no extra term because H = 4G).
struct CellWalk {
  int64_t hoff;
  int64_t zoff;
  int gx;

  LTHC_DEV void init(int64_t cell, int G, int C) {
    const int M = G * G;
    const int64_t H = static_cast<int64_t>(G) * kS;
    const int64_t b = cell / M;
    const int m = static_cast<int>(cell - b * M);
    const int gy = m / G;
    gx = m - gy * G;
    hoff = ((b * H + gy * kS) * H + gx * kS) * C;
    zoff = cell * C;
  }
  LTHC_DEV void next(int G, int C, int64_t row_skip) {
    zoff += C;
    hoff += kS * C;
    if (++gx == G) {
      gx = 0;
      hoff += row_skip;
    }
  }
};

#define LTHC_PHASE_BARRIER() __builtin_amdgcn_sched_barrier(0)

// Byte offset of tap (0, 0), channel 0 of a cell in the NHWC tensor: cell row
// r = cell / G starts 4 high-res rows (4*H*C elements) after row r - 1, and
// cell gx = cell % G starts 4*C elements into its tap row.
LTHC_DEV int64_t cell_hoff(int64_t cell, int G, int C) {
  const int64_t r = cell / G;
  return (r * (kS * kS) * G + (cell - r * G) * kS) * C;
}

// Grid-stride step of P cells over the NHWC tensor (byte offsets below 4 GiB)
// for any P, not only multiples of G, so a grid can fill every resident slot.
// P cells are P / G cell rows plus P % G cells; when the column of the current
// cell passes G the step crosses one more cell row, which adds the 3 high-res
// rows the column wrap skips (a cell row is 4 high-res rows, one of which the
// G column steps already cover).  `cell` is wave-uniform in every caller, so
// the column counter and the select live in scalar registers.
struct CellStride {
  uint32_t step_x;  // bytes of P / G cell rows plus P % G cells
  uint32_t wrap_x;  // 3 high-res rows
  uint32_t r;       // P % G
  uint32_t gx;      // column of the current cell
  uint32_t G;

  LTHC_DEV CellStride(uint32_t P, uint32_t cell, int G_, uint32_t tap_b, uint32_t row_b) {
    G = static_cast<uint32_t>(G_);
    r = P % G;
    gx = cell % G;
    step_x = (P / G) * kS * row_b + r * kS * tap_b;
    wrap_x = (kS - 1) * row_b;
  }
  // Bytes from the current cell to the one P cells on; moves the column.
  LTHC_DEV uint32_t advance() {
    gx += r;
    const bool wrap = gx >= G;
    gx = wrap ? gx - G : gx;
    return step_x + (wrap ? wrap_x : 0u);
  }
};

// ---------------------------------------------------------------------------
// READ: z[cell, c] = sum_k alpha[c,k] x[cell, k, c]
// Thread = VEC channels of one cell, all 16 taps; alpha for those channels
// lives in VGPRs.  Block = cpi cells x ncv_blk channel vectors.  Cells are
// visited grid-stride: the grid covers S = gridDim.x * cpi consecutive cells
// at a time (a compact window of the tensor, which HBM serves faster than
// one independent stream per block), and S % G == 0 makes every thread's
// byte offsets advance by constants.  Off is the byte-offset type (uint32_t
// when x is smaller than 4 GiB).
// Accumulation order k = 0..15 (local_thc_triton_kernels.py:51-55).
// ---------------------------------------------------------------------------
template <int DT, int WDT, int VEC, typename Off>
__global__ __launch_bounds__(kBlock) void read_fwd_kernel(const void* __restrict__ x, const void* __restrict__ w,
                                                          void* __restrict__ z, int64_t ncells, int G, int C,
                                                          int ncv_blk, int cpi) {
  constexpr int ES = Fmt<DT>::bytes;
  const int t = threadIdx.x;
  const int ci = t / ncv_blk;
  const int c0 = (blockIdx.y * ncv_blk + (t - ci * ncv_blk)) * VEC;
  int64_t cell = static_cast<int64_t>(blockIdx.x) * cpi + ci;
  if (ci >= cpi || c0 >= C || cell >= ncells) return;
  float a[VEC][kK];
#pragma unroll
  for (int v = 0; v < VEC; ++v) load_wvec<WDT, kK>(w, static_cast<int64_t>(c0 + v) * kK, a[v]);

  const Off row_b = static_cast<Off>(static_cast<int64_t>(G) * kS * C * ES);  // one high-res row, bytes
  const Off tap_b = static_cast<Off>(C * ES);
  const int64_t S = static_cast<int64_t>(gridDim.x) * cpi;
  const Off step_x = static_cast<Off>((S / G) * kS * row_b);
  const Off step_z = static_cast<Off>(S * C * ES);
  Off xo = static_cast<Off>((cell_hoff(cell, G, C) + c0) * ES);
  Off zo = static_cast<Off>((cell * C + c0) * ES);
  for (; cell < ncells; cell += S, xo += step_x, zo += step_z) {
    Raw<DT, VEC> xr[kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) load_at<DT, VEC, true>(x, xo + (k / kS) * row_b + (k % kS) * tap_b, xr[k]);
    LTHC_PHASE_BARRIER();
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      float xv[VEC];
      unpack_raw<DT, VEC>(xr[k], xv);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = fmaf(xv[v], a[v][k], acc[v]);
    }
    hold_f32<DT>(acc);  // rounded once from fp32 (no mixed-precision fp16 fma with the last product)
    store_at<DT, VEC>(z, zo, acc);
  }
}

// ---------------------------------------------------------------------------
// WHOLE-CELL MATERIALISE / WRITE (depth <= 24, tensors below 4 GiB):
// out[cell,k,c] = base[cell,k,c] + sum_l beta_l[c,k] dz_l[cell,c]
// Thread = CPT channels x the 16 / TG taps of its tap group (TG = 1: the
// whole cell; TG = 2: tap rows 0-1 or 2-3, for depths whose weights would
// not fit otherwise); its LMAX x CPT x (16 / TG) write weights stay in VGPRs.
// Block = TG groups x 256 / TG lanes, one slab of 256 * CPT / TG channels; a
// wavefront lies in one tap group, so each dz run is requested once per tap
// group (once per cell when TG = 1) and every wavefront access is a
// contiguous 64 * CPT-element run of one tap.  Cells are visited grid-stride
// with gridDim.x * gridDim.y equal to the resident block count (any gridDim.x:
// CellStride steps the offsets), so the whole grid sweeps one compact window
// of cells at a time with no tail round.  When L < LMAX (EXACT == false) the padding
// layers load layer 0 and contribute a selected 0.
// Accumulation: acc = base, acc = fma(beta_l, dz_l, acc) for l = 0..L-1
// (local_thc_triton_kernels.py:367-403).  Base reads and output writes are
// streaming (non-temporal).
// ---------------------------------------------------------------------------
template <int DT, int WDT, int LMAX, int CPT, int TG, bool HAS_BASE, bool EXACT>
__global__ __launch_bounds__(kBlock) void cell_mat_kernel(const void* __restrict__ base, PtrPack dz, PtrPack beta,
                                                          void* __restrict__ out, int L, uint32_t ncells, int G,
                                                          int C) {
  constexpr int ES = Fmt<DT>::bytes;
  constexpr int TPT = kK / TG;
  constexpr int QL = kBlock / TG;
  const int g = TG == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x / QL);  // wave-uniform tap group
  const int c0 = (blockIdx.y * QL + (threadIdx.x - g * QL)) * CPT;
  const int tap0 = g * TPT;
  uint32_t cell = blockIdx.x;
  if (c0 >= C || cell >= ncells) return;
  float bw[LMAX][CPT][TPT];
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    const void* bp = beta.p[(EXACT || l < L) ? l : 0];
#pragma unroll
    for (int v = 0; v < CPT; ++v) load_wvec<WDT, TPT>(bp, static_cast<int64_t>(c0 + v) * kK + tap0, bw[l][v]);
  }
  const uint32_t tap_b = C * ES;
  const uint32_t row_b = G * kS * tap_b;
  const uint32_t P = gridDim.x;
  CellStride stride(P, cell, G, tap_b, row_b);
  const uint32_t step_z = P * tap_b;
  uint32_t xo = static_cast<uint32_t>((cell_hoff(cell, G, C) + c0) * ES) + (tap0 / kS) * row_b;
  uint32_t zo = (cell * C + c0) * ES;
  for (; cell < ncells; cell += P, xo += stride.advance(), zo += step_z) {
    Raw<DT, CPT> xr[TPT];
    Raw<DT, CPT> dr[LMAX];
    if constexpr (HAS_BASE) {
#pragma unroll
      for (int k = 0; k < TPT; ++k) load_at<DT, CPT, true>(base, xo + (k / kS) * row_b + (k % kS) * tap_b, xr[k]);
    }
#pragma unroll
    for (int l = 0; l < LMAX; ++l) load_at<DT, CPT>(dz.p[(EXACT || l < L) ? l : 0], zo, dr[l]);
    LTHC_PHASE_BARRIER();

    float acc[TPT][CPT];
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
      if constexpr (HAS_BASE) {
        unpack_raw<DT, CPT>(xr[k], acc[k]);
      } else {
#pragma unroll
        for (int v = 0; v < CPT; ++v) acc[k][v] = 0.f;
      }
    }
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      float d[CPT];
      unpack_raw<DT, CPT>(dr[l], d);
      if constexpr (!EXACT) {
        const bool live = l < L;
#pragma unroll
        for (int v = 0; v < CPT; ++v) d[v] = live ? d[v] : 0.f;
      }
#pragma unroll
      for (int k = 0; k < TPT; ++k)
#pragma unroll
        for (int v = 0; v < CPT; ++v) acc[k][v] = fmaf(bw[l][v][k], d[v], acc[k][v]);
    }
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
      hold_f32<DT>(acc[k]);
      store_at<DT, CPT, true>(out, xo + (k / kS) * row_b + (k % kS) * tap_b, acc[k]);
    }
  }
}

// ---------------------------------------------------------------------------
// DEEP WHOLE-CELL MATERIALISE (depth 17-24 with a base, tensors below 4 GiB):
// cell_mat_kernel's thread (one channel x all 16 taps) for depths whose
// 16 x LMAX weights do not fit in VGPRs beside a cell's loads.  Layers
// 0..LV-1 keep their weights in VGPRs; layers LV..LMAX-1 are staged once per
// block into LDS as [layer][tap quad][channel] float4 rows, so a wavefront's
// read of one quad is 64 consecutive 16-byte lanes (no bank conflicts).
// Block = 4 wavefronts on one 64-channel slab, wavefront w on cell 4 b + w
// of each grid step (gridDim.x * 4 cells; NC = 2: cells 8 b + w and 8 b + w + 4
// of gridDim.x * 8, when 8 | G): each dz run is
// requested once per cell, where cell_mat_kernel's two tap groups request it
// twice at these depths.  Two cells per wavefront and step (NC = 2) put twice
// the loads in flight per wavefront and halve the LDS weight reads per cell
// (one quad read serves both cells); their registers leave room for 4 layers
// of weights in VGPRs, so 20 sit in LDS (80 KiB, two blocks per CU):
// 2 % faster than NC = 1 at configuration 5's shape, bitwise equal.  Same FMA order and roundings as cell_mat_kernel:
// acc = base, acc = fma(beta_l, dz_l, acc) for l = 0..L-1, one rounding.  When
// L < LMAX (EXACT == false) the padding layers' dz and beta entries point at
// layer 0 (filled in by the launcher, so the kernel indexes the pointer packs
// directly) and they contribute a selected 0, as in cell_mat_kernel; the
// layer count is re-read in every cell iteration, so the compiler does not
// hold a mask per layer across the loop (they spilled scalar registers).
// ---------------------------------------------------------------------------
template <int DT, int WDT, int LMAX, int LV, int NC, bool EXACT>
__global__ __launch_bounds__(kBlock, 2) void cell_mat_deep_kernel(const void* __restrict__ base, PtrPack dz,
                                                                  PtrPack beta, void* __restrict__ out, int L,
                                                                  uint32_t ncells, int G, int C) {
  constexpr int ES = Fmt<DT>::bytes;
  constexpr int LD = LMAX - LV;  // layers whose weights sit in LDS
  static_assert(LD >= 1 && LV >= 1, "layer split");
  static_assert(NC == 1 || NC == 2, "cells per wavefront and step");
  __shared__ float4 wl[LD][kK / 4][64];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c0 = blockIdx.y * 64 + lane;
  const bool live = c0 < C;  // every thread takes part in the staging and its barrier
#pragma unroll
  for (int j = 0; j < LD; ++j) {  // wavefront w stages tap quad w of every LDS layer
    const int l = LV + j;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (live) load_wvec<WDT, 4>(beta.p[l], static_cast<int64_t>(c0) * kK + 4 * w, v);
    wl[j][w][lane] = make_float4(v[0], v[1], v[2], v[3]);
  }
  float bw[LV][kK];
#pragma unroll
  for (int l = 0; l < LV; ++l) {
#pragma unroll
    for (int k = 0; k < kK; ++k) bw[l][k] = 0.f;
    if (live) load_wvec<WDT, kK>(beta.p[l], static_cast<int64_t>(c0) * kK, bw[l]);
  }
  __syncthreads();
  uint32_t cell = blockIdx.x * (4 * NC) + w;
  if (!live || cell >= ncells) return;
  const uint32_t tap_b = C * ES;
  const uint32_t row_b = G * kS * tap_b;
  const uint32_t P = gridDim.x * 4 * NC;
  CellStride stride(P, cell, G, tap_b, row_b);
  const uint32_t step_z = P * tap_b;
  // NC = 2: the wavefront's second cell is cell + 4, in the same cell row (the launcher requires 8 | G, so a block's
  // run of 8 cells starting at a multiple of 8 stays in one row, and 8 | ncells, so both cells exist)
  constexpr uint32_t kDn = 4;
  const uint32_t dxo = kDn * kS * tap_b, dzo = kDn * tap_b;
  uint32_t xo = static_cast<uint32_t>((cell_hoff(cell, G, C) + c0) * ES);
  uint32_t zo = (cell * C + c0) * ES;
  for (; cell < ncells; cell += P, xo += stride.advance(), zo += step_z) {
    Raw<DT, 1> xr[NC][kK];
    Raw<DT, 1> dr[NC][LMAX];
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int k = 0; k < kK; ++k)
        load_at<DT, 1, true>(base, xo + j * dxo + (k / kS) * row_b + (k % kS) * tap_b, xr[j][k]);
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int l = 0; l < LMAX; ++l) load_at<DT, 1>(dz.p[l], zo + j * dzo, dr[j][l]);
    LTHC_PHASE_BARRIER();

    float acc[NC][kK][1];
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int k = 0; k < kK; ++k) unpack_raw<DT, 1>(xr[j][k], acc[j][k]);
    int Lc = L;
    if constexpr (!EXACT) asm volatile("" : "+s"(Lc));
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      float d[NC][1];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        unpack_raw<DT, 1>(dr[j][l], d[j]);
        if constexpr (!EXACT) d[j][0] = l < Lc ? d[j][0] : 0.f;
      }
      if (l < LV) {
#pragma unroll
        for (int k = 0; k < kK; ++k)
#pragma unroll
          for (int j = 0; j < NC; ++j) acc[j][k][0] = fmaf(bw[l < LV ? l : 0][k], d[j][0], acc[j][k][0]);
      } else {
#pragma unroll
        for (int q = 0; q < kK / 4; ++q) {  // one LDS read of a tap quad serves the NC cells
          const float4 b = wl[l >= LV ? l - LV : 0][q][lane];
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            acc[j][4 * q + 0][0] = fmaf(b.x, d[j][0], acc[j][4 * q + 0][0]);
            acc[j][4 * q + 1][0] = fmaf(b.y, d[j][0], acc[j][4 * q + 1][0]);
            acc[j][4 * q + 2][0] = fmaf(b.z, d[j][0], acc[j][4 * q + 2][0]);
            acc[j][4 * q + 3][0] = fmaf(b.w, d[j][0], acc[j][4 * q + 3][0]);
          }
        }
      }
      if constexpr (NC == 2) LTHC_PHASE_BARRIER();  // one layer's LDS reads at a time (hoisted, they spilled)
    }
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int k = 0; k < kK; ++k) {
        hold_f32<DT>(acc[j][k]);
        store_at<DT, 1, true>(out, xo + j * dxo + (k / kS) * row_b + (k % kS) * tap_b, acc[j][k]);
      }
  }
}

// ---------------------------------------------------------------------------
// MATERIALISE / WRITE: out[cell,k,c] = base[cell,k,c] + sum_l beta_l[c,k] dz_l[cell,c]
// Thread = CPT channels x TPT taps of one tap row; its LMAX x CPT x TPT write
// weights stay in VGPRs.  Block = 256 threads = QS channel groups x NTG tap
// groups, covering all 16 taps of a CPT*QS channel slab; the block walks cpb
// consecutive cells, the cell position being uniform (scalar) across the
// block.  The NTG tap-group threads of a channel group load the same dz runs
// (L1 hits after the first).  When L < LMAX (EXACT == false) the padding
// layers load layer 0 and contribute a selected 0.
// Accumulation: acc = base, acc = fma(beta_l, dz_l, acc) for l = 0..L-1
// (local_thc_triton_kernels.py:367-403).  NT marks the base reads and the
// output writes as streaming, keeping L2 for the dz runs.
// ---------------------------------------------------------------------------
template <int DT, int WDT, int LMAX, int TPT, int CPT, bool HAS_BASE, bool EXACT, bool NT, typename Off>
__global__ __launch_bounds__(kBlock) void materialise_kernel(const void* __restrict__ base, PtrPack dz, PtrPack beta,
                                                             void* __restrict__ out, int L, int64_t ncells, int G,
                                                             int C, int64_t cpb) {
  constexpr int NTG = kK / TPT;
  constexpr int QS = kBlock / NTG;
  constexpr int ES = Fmt<DT>::bytes;
  const int t = threadIdx.x;
  const int g = t / QS;
  const int c0 = (blockIdx.y * QS + (t - g * QS)) * CPT;
  if (c0 >= C) return;
  const int tap0 = g * TPT;
  const int sy = tap0 / kS;
  const int sx0 = tap0 % kS;

  float bw[LMAX][CPT][TPT];
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    const void* bp = beta.p[(EXACT || l < L) ? l : 0];
#pragma unroll
    for (int v = 0; v < CPT; ++v) load_wvec<WDT, TPT>(bp, static_cast<int64_t>(c0 + v) * kK + tap0, bw[l][v]);
  }

  const int64_t H = static_cast<int64_t>(G) * kS;
  const Off lane_h = static_cast<Off>(((sy * H + sx0) * C + c0) * ES);
  const Off lane_z = static_cast<Off>(c0 * ES);
  const Off tap_b = static_cast<Off>(C * ES);
  const int64_t row_skip = 3 * H * C;
  const int64_t cb = static_cast<int64_t>(blockIdx.x) * cpb;
  const int64_t ce = std::min(ncells, cb + cpb);
  CellWalk cw;
  cw.init(cb, G, C);
  for (int64_t cell = cb; cell < ce; ++cell) {
    const Off xo = static_cast<Off>(cw.hoff * ES) + lane_h;
    const Off zo = static_cast<Off>(cw.zoff * ES) + lane_z;
    cw.next(G, C, row_skip);
    Raw<DT, CPT> xr[TPT];
    Raw<DT, CPT> dr[LMAX];
    if constexpr (HAS_BASE) {
#pragma unroll
      for (int j = 0; j < TPT; ++j) load_at<DT, CPT, NT>(base, xo + j * tap_b, xr[j]);
    }
#pragma unroll
    for (int l = 0; l < LMAX; ++l) load_at<DT, CPT>(dz.p[(EXACT || l < L) ? l : 0], zo, dr[l]);
    LTHC_PHASE_BARRIER();

    float acc[TPT][CPT];
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      if constexpr (HAS_BASE) {
        unpack_raw<DT, CPT>(xr[j], acc[j]);
      } else {
#pragma unroll
        for (int v = 0; v < CPT; ++v) acc[j][v] = 0.f;
      }
    }
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      float d[CPT];
      unpack_raw<DT, CPT>(dr[l], d);
      if constexpr (!EXACT) {
        const bool live = l < L;
#pragma unroll
        for (int v = 0; v < CPT; ++v) d[v] = live ? d[v] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < TPT; ++j)
#pragma unroll
        for (int v = 0; v < CPT; ++v) acc[j][v] = fmaf(bw[l][v][j], d[v], acc[j][v]);
    }
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      hold_f32<DT>(acc[j]);
      store_at<DT, CPT, NT>(out, xo + j * tap_b, acc[j]);
    }
  }
}

// ---------------------------------------------------------------------------
// MULTI-WEIGHT READ: out_l[cell,c] = sum_k w_l[c,k] g[cell,k,c]
// Thread = 4 channels x 16 taps x LC layers; the LC x 4 x 16 weights stay in
// VGPRs.  Block = QS quads x NLG layer groups (at most 256 threads); the NLG
// groups of a quad read the same g run (L1 hits after the first).
// Accumulation order k = 0..15 (local_thc_triton_kernels.py:580-592).
// ---------------------------------------------------------------------------
template <int DT, int WDT, int LC, typename Off>
__global__ __launch_bounds__(kBlock) void read_multi_kernel(const void* __restrict__ g, PtrPack w, PtrPack out, int L,
                                                            int QS, int64_t ncells, int G, int C, int64_t cpb) {
  constexpr int ES = Fmt<DT>::bytes;
  const int t = threadIdx.x;
  const int lg = t / QS;
  const int c0 = (blockIdx.y * QS + (t - lg * QS)) * 4;
  const int l0 = lg * LC;
  if (c0 >= C || l0 >= L) return;
  const int nl = std::min(LC, L - l0);

  float wr[LC][4][kK];
#pragma unroll
  for (int i = 0; i < LC; ++i) {
    const void* wp = w.p[l0 + (i < nl ? i : 0)];
#pragma unroll
    for (int v = 0; v < 4; ++v) load_wvec<WDT, kK>(wp, static_cast<int64_t>(c0 + v) * kK, wr[i][v]);
  }

  const int64_t H = static_cast<int64_t>(G) * kS;
  const Off row_b = static_cast<Off>(H * C * ES);
  const Off tap_b = static_cast<Off>(C * ES);
  const Off lane_c = static_cast<Off>(c0 * ES);
  const int64_t row_skip = 3 * H * C;
  const int64_t cb = static_cast<int64_t>(blockIdx.x) * cpb;
  const int64_t ce = std::min(ncells, cb + cpb);
  CellWalk cw;
  cw.init(cb, G, C);
  for (int64_t cell = cb; cell < ce; ++cell) {
    const Off go = static_cast<Off>(cw.hoff * ES) + lane_c;
    const Off zo = static_cast<Off>(cw.zoff * ES) + lane_c;
    cw.next(G, C, row_skip);
    Raw<DT, 4> gr[kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) load_at<DT, 4>(g, go + (k / kS) * row_b + (k % kS) * tap_b, gr[k]);
    LTHC_PHASE_BARRIER();
    float acc[LC][4];
#pragma unroll
    for (int i = 0; i < LC; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][v] = 0.f;
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      float gv[4];
      unpack_raw<DT, 4>(gr[k], gv);
#pragma unroll
      for (int i = 0; i < LC; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][v] = fmaf(gv[v], wr[i][v][k], acc[i][v]);
    }
#pragma unroll
    for (int i = 0; i < LC; ++i) {
      hold_f32<DT>(acc[i]);
      if (i < nl) store_at<DT, 4>(const_cast<void*>(out.p[l0 + i]), zo, acc[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// CELL WEIGHT GRADIENT, stage 1: per-block partial sums
//   partial[bx, l, c, k] = sum_{cells of block bx} high[cell,k,c] low_l[cell,c]
// Same thread mapping as materialise_kernel; the LMAX x TPT x CPT
// accumulators stay in VGPRs for the whole cell range of the block.  Padding
// layers (l >= L) accumulate layer 0 and are never written out.
// ---------------------------------------------------------------------------
template <int DT, int LMAX, int TPT, int CPT, bool NT, typename Off>
__global__ __launch_bounds__(kBlock) void wgrad_partial_kernel(const void* __restrict__ high, PtrPack low,
                                                               float* __restrict__ partial, int L, int64_t ncells,
                                                               int G, int C, int64_t cpb) {
  constexpr int NTG = kK / TPT;
  constexpr int QS = kBlock / NTG;
  constexpr int ES = Fmt<DT>::bytes;
  const int t = threadIdx.x;
  const int g = t / QS;
  const int c0 = (blockIdx.y * QS + (t - g * QS)) * CPT;
  if (c0 >= C) return;
  const int tap0 = g * TPT;
  const int sy = tap0 / kS;
  const int sx0 = tap0 % kS;

  float acc[LMAX][TPT][CPT];
#pragma unroll
  for (int l = 0; l < LMAX; ++l)
#pragma unroll
    for (int j = 0; j < TPT; ++j)
#pragma unroll
      for (int v = 0; v < CPT; ++v) acc[l][j][v] = 0.f;

  const int64_t H = static_cast<int64_t>(G) * kS;
  const Off lane_h = static_cast<Off>(((sy * H + sx0) * C + c0) * ES);
  const Off lane_z = static_cast<Off>(c0 * ES);
  const Off tap_b = static_cast<Off>(C * ES);
  const int64_t row_skip = 3 * H * C;
  const int64_t cb = static_cast<int64_t>(blockIdx.x) * cpb;
  const int64_t ce = std::min(ncells, cb + cpb);
  CellWalk cw;
  cw.init(cb, G, C);
  for (int64_t cell = cb; cell < ce; ++cell) {
    const Off ho = static_cast<Off>(cw.hoff * ES) + lane_h;
    const Off zo = static_cast<Off>(cw.zoff * ES) + lane_z;
    cw.next(G, C, row_skip);
    Raw<DT, CPT> hr[TPT];
    Raw<DT, CPT> dr[LMAX];
#pragma unroll
    for (int j = 0; j < TPT; ++j) load_at<DT, CPT, NT>(high, ho + j * tap_b, hr[j]);
#pragma unroll
    for (int l = 0; l < LMAX; ++l) load_at<DT, CPT>(low.p[l < L ? l : 0], zo, dr[l]);
    LTHC_PHASE_BARRIER();
    float h[TPT][CPT];
#pragma unroll
    for (int j = 0; j < TPT; ++j) unpack_raw<DT, CPT>(hr[j], h[j]);
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      float d[CPT];
      unpack_raw<DT, CPT>(dr[l], d);
#pragma unroll
      for (int j = 0; j < TPT; ++j)
#pragma unroll
        for (int v = 0; v < CPT; ++v) acc[l][j][v] = fmaf(h[j][v], d[v], acc[l][j][v]);
    }
  }
  float* dst = partial + static_cast<int64_t>(blockIdx.x) * L * C * kK;
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    if (l < L) {
#pragma unroll
      for (int v = 0; v < CPT; ++v) {
        float* row = dst + (static_cast<int64_t>(l) * C + c0 + v) * kK + tap0;
        if constexpr (TPT == 4) {
          *reinterpret_cast<float4*>(row) = make_float4(acc[l][0][v], acc[l][1][v], acc[l][2][v], acc[l][3][v]);
        } else {
#pragma unroll
          for (int j = 0; j < TPT; ++j) row[j] = acc[l][j][v];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// WHOLE-CELL MULTI-WEIGHT READ (depth <= 24, tensors below 4 GiB):
//   out_l[cell,c] = sum_k w_l[c,k] g[cell,k,c]
// Thread = CPT channels x all 16 taps x the LMAX / LG layers of its layer
// group; the weights stay in VGPRs.  Block = LG groups x 256 / LG lanes (a
// wavefront lies in one group), so each g run is loaded once per layer group
// (once per cell when LG = 1).  Grid and cell order as cell_mat_kernel.
// Padding layers (l >= L) load layer 0's weights and are never stored; with
// EXACT (L == LMAX) the kernel carries no layer masks.  The L outputs are
// written with streaming (non-temporal) stores, as are the materialise's.
// Accumulation order k = 0..15 (local_thc_triton_kernels.py:580-592).
// ---------------------------------------------------------------------------
template <int DT, int WDT, int LMAX, int CPT, int LG, bool EXACT>
__global__ __launch_bounds__(kBlock) void cell_read_multi_kernel(const void* __restrict__ g, PtrPack w, PtrPack out,
                                                                 int L, uint32_t ncells, int G, int C) {
  constexpr int ES = Fmt<DT>::bytes;
  constexpr int LPG = LMAX / LG;
  constexpr int QL = kBlock / LG;
  // the layer group is wave-uniform (QL >= 64): keep it scalar so out.p[l0 + i] is a scalar kernarg load
  const int lg = LG == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x / QL);
  const int c0 = (blockIdx.y * QL + (threadIdx.x - lg * QL)) * CPT;
  const int l0 = lg * LPG;
  uint32_t cell = blockIdx.x;
  if (c0 >= C || cell >= ncells || (!EXACT && l0 >= L)) return;
  float wr[LPG][CPT][kK];
#pragma unroll
  for (int i = 0; i < LPG; ++i)
#pragma unroll
    for (int v = 0; v < CPT; ++v)
      load_wvec<WDT, kK>(w.p[(EXACT || l0 + i < L) ? l0 + i : 0], static_cast<int64_t>(c0 + v) * kK, wr[i][v]);
  const uint32_t tap_b = C * ES;
  const uint32_t row_b = G * kS * tap_b;
  const uint32_t P = gridDim.x;
  CellStride stride(P, cell, G, tap_b, row_b);
  const uint32_t step_z = P * tap_b;
  uint32_t go = static_cast<uint32_t>((cell_hoff(cell, G, C) + c0) * ES);
  uint32_t zo = (cell * C + c0) * ES;
  for (; cell < ncells; cell += P, go += stride.advance(), zo += step_z) {
    Raw<DT, CPT> gr[kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) load_at<DT, CPT, true>(g, go + (k / kS) * row_b + (k % kS) * tap_b, gr[k]);
    LTHC_PHASE_BARRIER();
    float acc[LPG][CPT];
#pragma unroll
    for (int i = 0; i < LPG; ++i)
#pragma unroll
      for (int v = 0; v < CPT; ++v) acc[i][v] = 0.f;
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      float gv[CPT];
      unpack_raw<DT, CPT>(gr[k], gv);
#pragma unroll
      for (int i = 0; i < LPG; ++i)
#pragma unroll
        for (int v = 0; v < CPT; ++v) acc[i][v] = fmaf(gv[v], wr[i][v][k], acc[i][v]);
    }
#pragma unroll
    for (int i = 0; i < LPG; ++i) {
      hold_f32<DT>(acc[i]);
      if (EXACT || l0 + i < L) store_at<DT, CPT, true>(const_cast<void*>(out.p[l0 + i]), zo, acc[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// WHOLE-CELL CELL WEIGHT GRADIENT, stage 1 (depth <= 24, tensors below 4 GiB):
//   partial[bx, l, c, k] = sum_{cells of block bx} high[cell,k,c] low_l[cell,c]
// Thread = CPT channels x the 16 / TG taps of its tap group (as
// cell_mat_kernel); its LMAX x CPT x (16 / TG) fp32 accumulators stay in
// VGPRs.  A block's four wavefronts are TG tap groups x WC = 4 / TG cell
// lanes over the same 64 x CPT channels: cell lane w of block bx visits cells
// bx * WC + w, + WC * gridDim.x, ...  At the end the WC cell lanes are added
// in lane order through LDS, so each block writes one partial slot (zeros
// included) -- WC times fewer partial bytes than a slot per wavefront.
// Padding layers accumulate layer 0 and are never written.
// ---------------------------------------------------------------------------
template <int DT, int LMAX, int CPT, int TG>
__global__ __launch_bounds__(kBlock) void cell_wgrad_kernel(const void* __restrict__ high, PtrPack low,
                                                            float* __restrict__ partial, int L, uint32_t ncells, int G,
                                                            int C) {
  constexpr int ES = Fmt<DT>::bytes;
  constexpr int TPT = kK / TG;
  constexpr int WC = 4 / TG;                  // cell lanes per tap group
  constexpr int PER = CPT * TPT;              // accumulators per layer
  constexpr int LC = 64 / PER < 1 ? 1 : (64 / PER > LMAX ? LMAX : 64 / PER);  // layers per LDS round
  constexpr int SLOTS = LC * PER / 4;         // float4 per lane per round
  static_assert(PER % 4 == 0 && LMAX % LC == 0, "weight-gradient reduction rounds");
  __shared__ float4 red[(WC - 1) * TG][SLOTS][64];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = w % TG, cw = w / TG;
  const int c0 = (blockIdx.y * 64 + lane) * CPT;
  const int tap0 = g * TPT;
  const bool active = c0 < C;  // every thread reaches the reduction's barriers
  float acc[LMAX][CPT][TPT];
#pragma unroll
  for (int l = 0; l < LMAX; ++l)
#pragma unroll
    for (int v = 0; v < CPT; ++v)
#pragma unroll
      for (int k = 0; k < TPT; ++k) acc[l][v][k] = 0.f;
  const uint32_t tap_b = C * ES;
  const uint32_t row_b = G * kS * tap_b;
  const uint32_t P = gridDim.x * WC;  // cell stride
  const uint32_t step_z = P * tap_b;
  uint32_t cell = active ? blockIdx.x * WC + cw : ncells;
  CellStride stride(P, cell < ncells ? cell : 0, G, tap_b, row_b);
  uint32_t ho = static_cast<uint32_t>((cell_hoff(cell < ncells ? cell : 0, G, C) + c0) * ES) + (tap0 / kS) * row_b;
  uint32_t zo = (cell * C + c0) * ES;
  for (; cell < ncells; cell += P, ho += stride.advance(), zo += step_z) {
    Raw<DT, CPT> hr[TPT];
    Raw<DT, CPT> dr[LMAX];
#pragma unroll
    for (int k = 0; k < TPT; ++k) load_at<DT, CPT, true>(high, ho + (k / kS) * row_b + (k % kS) * tap_b, hr[k]);
#pragma unroll
    for (int l = 0; l < LMAX; ++l) load_at<DT, CPT>(low.p[l < L ? l : 0], zo, dr[l]);
    LTHC_PHASE_BARRIER();
    float h[TPT][CPT];
#pragma unroll
    for (int k = 0; k < TPT; ++k) unpack_raw<DT, CPT>(hr[k], h[k]);
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      float d[CPT];
      unpack_raw<DT, CPT>(dr[l], d);
#pragma unroll
      for (int v = 0; v < CPT; ++v)
#pragma unroll
        for (int k = 0; k < TPT; ++k) acc[l][v][k] = fmaf(h[k][v], d[v], acc[l][v][k]);
    }
  }
  float* dst = partial + static_cast<int64_t>(blockIdx.x) * L * C * kK;
#pragma unroll
  for (int l0 = 0; l0 < LMAX; l0 += LC) {
    if (cw > 0) {
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) {
        const int e = 4 * q;  // element e of the round: layer l0 + e / PER, channel (e % PER) / TPT, taps e % TPT + 0..3
        const int l = l0 + e / PER, v = (e % PER) / TPT, k = e % TPT;
        red[(cw - 1) * TG + g][q][lane] = make_float4(acc[l][v][k], acc[l][v][k + 1], acc[l][v][k + 2], acc[l][v][k + 3]);
      }
    }
    __syncthreads();
    if (cw == 0 && active) {
#pragma unroll
      for (int q = 0; q < SLOTS; ++q) {
        const int e = 4 * q;
        const int l = l0 + e / PER, v = (e % PER) / TPT, k = e % TPT;
        float4 t = make_float4(acc[l][v][k], acc[l][v][k + 1], acc[l][v][k + 2], acc[l][v][k + 3]);
#pragma unroll
        for (int r = 1; r < WC; ++r) {
          const float4 b = red[(r - 1) * TG + g][q][lane];
          t.x += b.x;
          t.y += b.y;
          t.z += b.z;
          t.w += b.w;
        }
        if (l < L) *reinterpret_cast<float4*>(dst + (static_cast<int64_t>(l) * C + c0 + v) * kK + tap0 + k) = t;
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

// Stage 2: out[i] = sum_{p < nparts} partial[p, i] in ascending p, stored in
// format odt (the fp32 sum rounded once).
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ partial, int nparts,
                                                              int64_t n, void* __restrict__ out, int odt) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int p = 0; p < nparts; ++p) s += partial[static_cast<int64_t>(p) * n + i];
  store_w(out, odt, i, s);
}

// Narrow outputs (few columns, many partial rows): block = 16 columns x 16
// part groups; group g sums parts g, g + 16, g + 32, ... in order, then the
// 16 group sums are added in order g = 0..15 -- a fixed order, so the result
// is bitwise reproducible, with 16x the parallelism of reduce_partials_kernel.
constexpr int kRedGroups = 16;
// A 256-thread block reduces COLS consecutive columns with 256 / COLS part groups: group g sums parts g, g + NG,
// g + 2 NG, ... in order (NG = 256 / COLS), then the group sums are added in order g = 0..NG-1.  COLS = 16 gives 16
// groups (narrow outputs: many partial rows over few columns); COLS = 64 makes a wavefront's load one 256-byte run
// of a partial row (wide outputs).
template <int COLS>
__device__ __forceinline__ void reduce_split_block(const float* __restrict__ partial, int nparts, int64_t n,
                                                   int64_t cblock, void* __restrict__ out, int odt) {
  constexpr int NG = 256 / COLS;
  __shared__ float part[NG][COLS];
  const int col = threadIdx.x % COLS;
  const int grp = threadIdx.x / COLS;
  const int64_t i = cblock * COLS + col;
  float s = 0.f;
  if (i < n) {
    // loads in batches of 8 (in flight together), added in part order
    int p = grp;
    for (; p + 7 * NG < nparts; p += 8 * NG) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = partial[static_cast<int64_t>(p + j * NG) * n + i];
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
    }
    for (; p < nparts; p += NG) s += partial[static_cast<int64_t>(p) * n + i];
  }
  part[grp][col] = s;
  __syncthreads();
  if (grp == 0 && i < n) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) t += part[g][col];
    store_w(out, odt, i, t);
  }
}

template <int COLS>
__global__ __launch_bounds__(256) void reduce_partials_split_kernel(const float* __restrict__ partial, int nparts,
                                                                    int64_t n, void* __restrict__ out, int odt) {
  reduce_split_block<COLS>(partial, nparts, n, blockIdx.x, out, odt);
}

// Several independent reductions in one launch (fp32 outputs), each segment's columns summed as
// reduce_partials_split_kernel<16> sums them (16-column blocks: the 64-column form measured slower here, where
// the segments have few partial rows).
struct RedSeg {
  const float* partial;
  float* out;
  int64_t n;
  int64_t block0;  // first block of the segment
  int nparts;
};
constexpr int kRedMaxSegs = 4;
struct RedSegs {
  RedSeg s[kRedMaxSegs];
  int nseg;
};

__global__ __launch_bounds__(256) void reduce_partials_multi_kernel(RedSegs segs) {
  const int64_t b = blockIdx.x;
  int si = 0;
  while (si + 1 < segs.nseg && b >= segs.s[si + 1].block0) ++si;
  const RedSeg& sg = segs.s[si];
  reduce_split_block<16>(sg.partial, sg.nparts, sg.n, b - sg.block0, sg.out, LTHC_F32);
}

// ---------------------------------------------------------------------------
// GAMMA: gamma[l, c] = sum_k alpha[c,k] beta_l[c,k], k = 0..K-1 in order
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gamma_kernel(const void* __restrict__ alpha, PtrPack beta, int wdt,
                                                    void* __restrict__ gamma, int odt, int C, int K, int L) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(L) * C) return;
  const int l = static_cast<int>(i / C);
  const int c = static_cast<int>(i - static_cast<int64_t>(l) * C);
  float s = 0.f;
  for (int k = 0; k < K; ++k)
    s = fmaf(load_w(alpha, wdt, static_cast<int64_t>(c) * K + k), load_w(beta.p[l], wdt, static_cast<int64_t>(c) * K + k), s);
  store_w(gamma, odt, i, s);
}

// The same for K == 16 and 16-byte aligned rows: each row is one vector load
// (four for fp32), all issued before the 16 FMAs (the k order is unchanged).
template <int WDT, int ODT>
__global__ __launch_bounds__(256) void gamma16_kernel(const void* __restrict__ alpha, PtrPack beta,
                                                      void* __restrict__ gamma, int C, int L) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(L) * C) return;
  const int l = static_cast<int>(i / C);
  const int c = static_cast<int>(i - static_cast<int64_t>(l) * C);
  float a[kK], b[kK];
  load_wvec<WDT, kK>(alpha, static_cast<int64_t>(c) * kK, a);
  load_wvec<WDT, kK>(beta.p[l], static_cast<int64_t>(c) * kK, b);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kK; ++k) s = fmaf(a[k], b[k], s);
  store_w(gamma, ODT, i, s);
}

// ---------------------------------------------------------------------------
// GAMMA with the eager dtype sequence (LayerLocalWrite.gamma_from_alpha under
// autocast, local_thc.py:1278-1283 with alpha cast at :1326):
//   gamma[l, c] = r(sum_k r(r(alpha[c,k]) * r(beta_l[c,k])))   sum in fp32, k = 0..K-1
// r = round to the output dtype (identity for fp32).
// ---------------------------------------------------------------------------
template <int ODT>
__global__ __launch_bounds__(256) void gamma_rounded_kernel(const void* __restrict__ alpha, int adt, PtrPack beta,
                                                            int bdt, void* __restrict__ gamma, int C, int K, int L) {
#pragma clang fp contract(off)  // the product is rounded before it is summed
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(L) * C) return;
  const int l = static_cast<int>(i / C);
  const int c = static_cast<int>(i - static_cast<int64_t>(l) * C);
  float s = 0.f;
  for (int k = 0; k < K; ++k) {
    const float a = round_w<ODT>(load_w(alpha, adt, static_cast<int64_t>(c) * K + k));
    const float b = round_w<ODT>(load_w(beta.p[l], bdt, static_cast<int64_t>(c) * K + k));
    s += round_w<ODT>(a * b);
  }
  store_w(gamma, ODT, i, s);
}

// The same for K = 16 taps with 16-byte aligned rows: one vector load per row,
// compile-time dtypes, the same rounding and summation order.
template <int ODT, int ADT, int BDT>
__global__ __launch_bounds__(256) void gamma16_rounded_kernel(const void* __restrict__ alpha, PtrPack beta,
                                                              void* __restrict__ gamma, int C, int L) {
#pragma clang fp contract(off)
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(L) * C) return;
  const int l = static_cast<int>(i / C);
  const int c = static_cast<int>(i - static_cast<int64_t>(l) * C);
  float a[kK], b[kK];
  load_wvec<ADT, kK>(alpha, static_cast<int64_t>(c) * kK, a);
  load_wvec<BDT, kK>(beta.p[l], static_cast<int64_t>(c) * kK, b);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kK; ++k) s += round_w<ODT>(round_w<ODT>(a[k]) * round_w<ODT>(b[k]));
  store_w(gamma, ODT, i, s);
}

// Its backward, the eager autograd of that sequence: with a = r(alpha),
// b_l = r(beta_l) and g_l = grad[l, c],
//   gbeta_l[c,k] = r(g_l * a[c,k])
//   galpha[c,k]  = r(... r(r(g_{L-1} b_{L-1}) + r(g_{L-2} b_{L-2})) ... + r(g_0 b_0))
// the L products being summed into a's gradient in the order autograd
// delivers them (last layer first), each partial sum rounded.
// Blocks [0, nb_beta) write gbeta, one thread per (l, c, k); the blocks after
// them write galpha, one thread per (c, k) over the L layers.
template <int ODT, int BDT, int LMAX>
__global__ __launch_bounds__(256) void gamma_rounded_bwd_kernel(const void* __restrict__ grad,
                                                                const void* __restrict__ alpha, int adt,
                                                                PtrPack beta, void* __restrict__ galpha,
                                                                PtrPack gbeta, int C, int K, int L, int nb_beta) {
#pragma clang fp contract(off)
  const int64_t n = static_cast<int64_t>(C) * K;
  if (static_cast<int>(blockIdx.x) < nb_beta) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (j >= n * L) return;
    const int l = static_cast<int>(j / n);
    const int64_t i = j - l * n;
    if (gbeta.p[l] == nullptr) return;
    const float g = load_w(grad, ODT, static_cast<int64_t>(l) * C + i / K);
    const float a = round_w<ODT>(load_w(alpha, adt, i));
    store_w(const_cast<void*>(gbeta.p[l]), BDT, i, round_w<ODT>(g * a));
    return;
  }
  const int64_t i = static_cast<int64_t>(blockIdx.x - nb_beta) * 256 + threadIdx.x;
  if (i >= n || galpha == nullptr) return;
  const int c = static_cast<int>(i / K);
  // every layer's loads first, unconditional so that they are in flight together (padding layers
  // l >= L load layer 0 and are not used), then the products
  float gv[LMAX], bv[LMAX];
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    const int ll = l < L ? l : 0;
    float g1[1], b1[1];
    load_wvec<ODT, 1>(grad, static_cast<int64_t>(ll) * C + c, g1);
    load_wvec<BDT, 1>(beta.p[ll], i, b1);
    gv[l] = g1[0];
    bv[l] = round_w<ODT>(b1[0]);
  }
  float acc = 0.f;
#pragma unroll
  for (int l = LMAX - 1; l >= 0; --l) {
    if (l < L) {
      const float pa = round_w<ODT>(gv[l] * bv[l]);
      acc = l == L - 1 ? pa : round_w<ODT>(acc + pa);
    }
  }
  store_w(galpha, adt, i, acc);
}

// ---------------------------------------------------------------------------
// RECURRENCE: z_next = fma(gamma, dz, z).  Block = 64 channel quads x 4 row
// lanes; each thread keeps its 4 gammas.  A block handles chunks of 4 * RU
// consecutive rows, grid-stride over the chunks, RU rows per phase (loads of
// rows past the end are clamped to the last row and their results dropped).
// ---------------------------------------------------------------------------
constexpr int kRU = 4;
// The backward's rows per phase: 2 measured faster than 4 at every size (B=64, C=768 -2.7 %; configuration 5 -1 %;
// B=256 -8.5 %; gdz and the summed gradient bitwise equal), 8 slower except at C=1024.  Lanes of 8 channels
// (16 bytes) with blocks of whole rows were slower at C=768.
constexpr int kRUB = 2;

template <int DT, typename Off>
__global__ __launch_bounds__(256) void recur_fwd_kernel(const void* __restrict__ z, const void* __restrict__ dz,
                                                        const void* __restrict__ gamma, int gdt,
                                                        void* __restrict__ zn, int64_t rows, int C) {
  constexpr int ES = Fmt<DT>::bytes;
  const int t = threadIdx.x;
  const int c0 = (blockIdx.x * 64 + (t & 63)) * 4;
  if (c0 >= C) return;
  float gm[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) gm[v] = load_w(gamma, gdt, c0 + v);
  // grid-stride over chunks of 4 * kRU rows: block y owns chunks y, y + gridDim.y, ...
  const int64_t re = rows;
  const int64_t S = static_cast<int64_t>(4 * kRU) * gridDim.y;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.y) * 4 * kRU + (t >> 6); r0 < re; r0 += S) {
    Raw<DT, 4> ar[kRU], dr[kRU];
    Off off[kRU];
#pragma unroll
    for (int u = 0; u < kRU; ++u) {
      const int64_t r = std::min(r0 + 4 * u, re - 1);
      off[u] = static_cast<Off>((r * C + c0) * ES);
      load_at<DT, 4>(z, off[u], ar[u]);
      load_at<DT, 4>(dz, off[u], dr[u]);
    }
    LTHC_PHASE_BARRIER();
#pragma unroll
    for (int u = 0; u < kRU; ++u) {
      float a[4], d[4];
      unpack_raw<DT, 4>(ar[u], a);
      unpack_raw<DT, 4>(dr[u], d);
#pragma unroll
      for (int v = 0; v < 4; ++v) a[v] = fmaf(gm[v], d[v], a[v]);
      if (r0 + 4 * u < re) store_at<DT, 4>(zn, off[u], a);
    }
  }
}

// ---------------------------------------------------------------------------
// RECURRENCE, one-shot form (16-byte lanes, tensors below 4 GiB): thread i
// owns elements [VEC*i, VEC*i + VEC) of the flattened [rows, C] tensors
// (C % VEC == 0, so the run lies in one row); one launch covers every run.
// Blocks are dispatched in order, so the resident blocks sweep one compact
// window of the three tensors: 6 % faster than the grid-stride form over a
// chain of 12 steps at the metric shape, same results bit for bit.
// ---------------------------------------------------------------------------
template <int DT, int GDT>
__global__ __launch_bounds__(256) void recur_fwd_flat_kernel(const void* __restrict__ z, const void* __restrict__ dz,
                                                             const void* __restrict__ gamma, void* __restrict__ zn,
                                                             uint32_t nvec, uint32_t cvec) {
  constexpr int ES = Fmt<DT>::bytes;
  constexpr int VEC = 16 / ES;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= nvec) return;
  const uint32_t c0 = (i % cvec) * VEC;
  const uint32_t off = i * 16u;
  Raw<DT, VEC> ar, dr;
  load_at<DT, VEC>(z, off, ar);
  load_at<DT, VEC>(dz, off, dr);
  float g[VEC];
  load_wvec<GDT, VEC>(gamma, c0, g);
  float a[VEC], d[VEC];
  unpack_raw<DT, VEC>(ar, a);
  unpack_raw<DT, VEC>(dr, d);
#pragma unroll
  for (int v = 0; v < VEC; ++v) a[v] = fmaf(g[v], d[v], a[v]);
  store_at<DT, VEC>(zn, off, a);
}

// RECURRENCE BACKWARD: gdz = gamma * g (+ gadd, HAS_ADD); partial[by, c] = sum
// g*dz over the rows the block visits (each thread's rows summed in its
// order, then the block's 4 row lanes added in lane order).  Grid and row
// order as recur_fwd_kernel.  HAS_G2: g is the sum of two gradients, g + g2 rounded to
// DT (the value of autograd's add of the two), which is also written to gsum.
template <int DT, typename Off, bool HAS_ADD, bool HAS_G2 = false>
__global__ __launch_bounds__(256) void recur_bwd_kernel(const void* __restrict__ g, const void* __restrict__ dz,
                                                        const void* __restrict__ gadd,
                                                        const void* __restrict__ gamma, int gdt,
                                                        void* __restrict__ gdz, float* __restrict__ partial,
                                                        int64_t rows, int C, const void* __restrict__ g2 = nullptr,
                                                        void* __restrict__ gsum = nullptr) {
  constexpr int ES = Fmt<DT>::bytes;
  const int t = threadIdx.x;
  const int c0 = (blockIdx.x * 64 + (t & 63)) * 4;
  const bool active = c0 < C;  // every thread reaches the block reduction below
  float gm[4] = {0.f, 0.f, 0.f, 0.f};
  if (active) {
#pragma unroll
    for (int v = 0; v < 4; ++v) gm[v] = load_w(gamma, gdt, c0 + v);
  }
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  const int64_t re = active ? rows : 0;
  const int64_t S = static_cast<int64_t>(4 * kRUB) * gridDim.y;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.y) * 4 * kRUB + (t >> 6); r0 < re; r0 += S) {
    Raw<DT, 4> ar[kRUB], dr[kRUB], xr[HAS_ADD ? kRUB : 1], br[HAS_G2 ? kRUB : 1];
    Off off[kRUB];
#pragma unroll
    for (int u = 0; u < kRUB; ++u) {
      const int64_t r = std::min(r0 + 4 * u, re - 1);
      off[u] = static_cast<Off>((r * C + c0) * ES);
      load_at<DT, 4, true>(g, off[u], ar[u]);
      if constexpr (HAS_G2) load_at<DT, 4, true>(g2, off[u], br[u]);
      load_at<DT, 4, true>(dz, off[u], dr[u]);
      if constexpr (HAS_ADD) load_at<DT, 4, true>(gadd, off[u], xr[u]);
    }
    LTHC_PHASE_BARRIER();
#pragma unroll
    for (int u = 0; u < kRUB; ++u) {
      if (r0 + 4 * u < re) {
        float a[4], d[4], o4[4];
        unpack_raw<DT, 4>(ar[u], a);
        if constexpr (HAS_G2) {
          float b[4];
          unpack_raw<DT, 4>(br[u], b);
#pragma unroll
          for (int v = 0; v < 4; ++v) a[v] += b[v];
          Raw<DT, 4> sr;  // the sum rounded to DT, stored and used from here on
          if constexpr (DT == LTHC_F32) {
#pragma unroll
            for (int v = 0; v < 4; ++v) sr.w[v] = __float_as_uint(a[v]);
          } else {
            sr.w[0] = pack2<DT>(a[0], a[1]);
            sr.w[1] = pack2<DT>(a[2], a[3]);
          }
          unpack_raw<DT, 4>(sr, a);
          store_at<DT, 4, true>(gsum, off[u], a);
        }
        unpack_raw<DT, 4>(dr[u], d);
        if constexpr (HAS_ADD) {
          unpack_raw<DT, 4>(xr[u], o4);
#pragma unroll
          for (int v = 0; v < 4; ++v) o4[v] = fmaf(gm[v], a[v], o4[v]);
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) o4[v] = gm[v] * a[v];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) s[v] = fmaf(a[v], d[v], s[v]);
        store_at<DT, 4, true>(gdz, off[u], o4);
      }
    }
  }
  __shared__ float4 lane_sum[4][64];
  lane_sum[t >> 6][t & 63] = make_float4(s[0], s[1], s[2], s[3]);
  __syncthreads();
  if (t < 64 && active) {
    float4 a = lane_sum[0][t];
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      const float4 b = lane_sum[q][t];
      a.x += b.x;
      a.y += b.y;
      a.z += b.z;
      a.w += b.w;
    }
    *reinterpret_cast<float4*>(partial + static_cast<int64_t>(blockIdx.y) * C + c0) = a;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
thread_local std::string g_last_error;

int fail(int code, const char* fn, const std::string& msg) {
  g_last_error = std::string(fn) + ": " + msg;
  return code;
}

int check_launch(const char* fn) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LTHC_ERR_HIP, fn, std::string("kernel launch failed: ") + hipGetErrorString(e));
  return LTHC_OK;
}

int num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

bool valid_dtype(int dt) { return dt == LTHC_F32 || dt == LTHC_BF16 || dt == LTHC_F16; }
int esize(int dt) { return dt == LTHC_F32 ? 4 : 2; }
bool aligned(const void* p, int64_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

int check_geom(const char* fn, int64_t B, int64_t G, int64_t s, int64_t C) {
  if (B < 0) return fail(LTHC_ERR_INVALID, fn, "B must be >= 0");
  if (G <= 0 || C <= 0) return fail(LTHC_ERR_INVALID, fn, "G and C must be positive");
  if (s != kS) return fail(LTHC_ERR_UNSUPPORTED, fn, "only cell side s == 4 (16 taps) is implemented");
  if (C % 4 != 0) return fail(LTHC_ERR_INVALID, fn, "C must be a multiple of 4");
  if (G > 4096 || C > (1 << 24)) return fail(LTHC_ERR_INVALID, fn, "G or C out of range");
  if (B > (int64_t(1) << 40) / (G * G * kK * C)) return fail(LTHC_ERR_INVALID, fn, "tensor too large");
  return LTHC_OK;
}

int check_act(const char* fn, const void* p, int dt, const char* name) {
  if (p == nullptr) return fail(LTHC_ERR_INVALID, fn, std::string(name) + " is NULL");
  if (!aligned(p, 4 * esize(dt))) return fail(LTHC_ERR_INVALID, fn, std::string(name) + " is not aligned to 4 elements");
  return LTHC_OK;
}

// Weights are read as whole 16-tap rows: 16-byte alignment.
int check_weight(const char* fn, const void* p, const std::string& name) {
  if (p == nullptr) return fail(LTHC_ERR_INVALID, fn, name + " is NULL");
  if (!aligned(p, 16)) return fail(LTHC_ERR_INVALID, fn, name + " is not 16-byte aligned");
  return LTHC_OK;
}

// Activation / weight dtype pairs with compiled kernels: weights in fp32 or
// in the activation dtype.
bool supported_pair(int x_dtype, int w_dtype) { return w_dtype == LTHC_F32 || w_dtype == x_dtype; }

// Cells per block so that a launch has about `blocks_per_cu` blocks per CU.
int64_t cells_per_block(int64_t ncells, int64_t slabs, int blocks_per_cu) {
  const int64_t target = std::max<int64_t>(1, static_cast<int64_t>(num_cus()) * blocks_per_cu / std::max<int64_t>(1, slabs));
  return std::max<int64_t>(1, (ncells + target - 1) / target);
}

// Grid-stride cell sweeps need the cells covered per grid step to be a
// multiple of G (constant offset increments) and of `cpi` (cells per block).
// Returns the step closest below `want` cells, at least one such multiple and
// at most ncells rounded up.
int64_t grid_step_cells(int64_t want, int64_t ncells, int G, int cpi) {
  const int64_t unit = std::lcm<int64_t>(G, cpi);
  const int64_t cap = (ncells + unit - 1) / unit * unit;
  return std::max<int64_t>(unit, std::min<int64_t>(want / unit * unit, cap));
}

// Cells per grid step of the kernels that step with CellStride (any multiple
// of `cpi`, the cells per block): `want`, the resident capacity in cells,
// rounded down to a multiple of cpi, at least cpi and at most ncells rounded
// up.  Every resident slot is used (rounding the step to a multiple of G left
// 10 of 170 blocks per slab empty at 256 CUs, two blocks per CU and 3 slabs).
int64_t grid_cells(int64_t want, int64_t ncells, int cpi) {
  const int64_t cap = (ncells + cpi - 1) / cpi * cpi;
  return std::max<int64_t>(cpi, std::min<int64_t>(want / cpi * cpi, cap));
}

// Shape of the whole-cell kernels per depth bucket: channels per thread CPT
// and groups per block GR (tap groups of the materialise / weight gradient,
// layer groups of the multi-weight read).  The LMAX x CPT x 16 / GR fp32
// weights (or accumulators), one cell's loads and the accumulators fit in
// 256 VGPRs: one group up to depth 12, two up to depth 24.
template <int DT, int LMAX>
struct CellMatShape {
  static constexpr int CPT = DT == LTHC_F32 ? (LMAX <= 1 ? 2 : 1) : (LMAX <= 1 ? 4 : (LMAX <= 4 ? 2 : 1));
  static constexpr int GR = LMAX <= 12 ? 1 : 2;
};

// Depth buckets of the whole-cell kernels.
constexpr int kCellMaxDepth = 24;

// Blocks of `kernel` (kBlock threads) resident on one CU.
template <typename K>
int resident_blocks(K kernel) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kBlock, 0) != hipSuccess || n < 1) n = 1;
  return n;
}

// Recurrence forward: row chunks (of 4 * kRU rows) in flight per channel
// block column, measured best at 1024 on MI355X.  Backward: 256 (each block
// row leaves one partial row of C floats to reduce).
const int64_t kRecurChunks = 1024;
const int64_t kRecurBwdChunks = 256;

int64_t recur_bwd_blocks_y(int64_t rows) { return std::min((rows + 4 * kRUB - 1) / (4 * kRUB), kRecurBwdChunks); }

// Deterministic reduction of nparts partial rows of n floats into out.
void launch_reduce(const float* partial, int nparts, int64_t n, void* out, hipStream_t st, int odt = LTHC_F32) {
  if (nparts <= kRedGroups) {
    reduce_partials_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(partial, nparts, n, out, odt);
  } else if (n >= 64 * 256) {  // wide: 64-column blocks (a wavefront's load is one 256-byte run of a partial row)
    reduce_partials_split_kernel<64><<<static_cast<unsigned>((n + 63) / 64), 256, 0, st>>>(partial, nparts, n, out, odt);
  } else {
    reduce_partials_split_kernel<16><<<static_cast<unsigned>((n + 15) / 16), 256, 0, st>>>(partial, nparts, n, out, odt);
  }
}

// The reductions of up to kRedMaxSegs (partial, nparts, n, out) segments in one launch.
void launch_reduce_multi(std::initializer_list<RedSeg> list, hipStream_t st) {
  RedSegs segs{};
  int64_t blocks = 0;
  for (const RedSeg& r : list) {
    RedSeg& d = segs.s[segs.nseg++];
    d = r;
    d.block0 = blocks;
    blocks += (r.n + 15) / 16;
  }
  reduce_partials_multi_kernel<<<static_cast<unsigned>(blocks), 256, 0, st>>>(segs);
}

template <int V>
using IC = std::integral_constant<int, V>;

template <typename T>
struct TypeTag {
  using type = T;
};

// Calls f(IC<DT>, IC<WDT>) for a supported (activation, weight) dtype pair.
template <typename F>
void dispatch_pair(int xdt, int wdt, F&& f) {
  switch (xdt) {
    case LTHC_F32: f(IC<LTHC_F32>{}, IC<LTHC_F32>{}); break;
    case LTHC_BF16:
      if (wdt == LTHC_F32) f(IC<LTHC_BF16>{}, IC<LTHC_F32>{});
      else f(IC<LTHC_BF16>{}, IC<LTHC_BF16>{});
      break;
    default:
      if (wdt == LTHC_F32) f(IC<LTHC_F16>{}, IC<LTHC_F32>{});
      else f(IC<LTHC_F16>{}, IC<LTHC_F16>{});
      break;
  }
}

template <typename F>
void dispatch_dtype(int dt, F&& f) {
  switch (dt) {
    case LTHC_F32: f(IC<LTHC_F32>{}); break;
    case LTHC_BF16: f(IC<LTHC_BF16>{}); break;
    default: f(IC<LTHC_F16>{}); break;
  }
}

// 32-bit byte offsets when every tensor of the call is below 4 GiB.
bool fits32(int64_t bytes) { return bytes < (int64_t(1) << 32); }

template <typename F>
void dispatch_off(bool off32, F&& f) {
  if (off32) f(TypeTag<uint32_t>{});
  else f(TypeTag<int64_t>{});
}

// Launch plan of the weight-gradient kernels, shared with the workspace query.
struct WgradPlan {
  bool cell;     // whole-cell grid-stride kernel (depth <= 12, tensors below 4 GiB)
  int tpt;       // taps per thread of the block-range kernel
  int slabs;     // channel slabs (grid y)
  int64_t cpb;   // cells per block of the block-range kernel
  int64_t nbx;   // blocks per slab = partial slots
};

template <int LMAX>
struct CellShape;

// (TPT, CPT) of the block-range weight-gradient kernel for depth L (the CellShape bucket).
void wgrad_shape(int L, int& tpt, int& cpt);

template <int DT, int LMAX>
void cell_wgrad_plan_l(WgradPlan& p, int64_t ncells, int G, int64_t C) {
  constexpr int CPT = CellMatShape<DT, LMAX>::CPT, GR = CellMatShape<DT, LMAX>::GR;
  constexpr int WC = 4 / GR;  // cell lanes per block (the cell stride is nbx * WC)
  static const int per_cu = resident_blocks(cell_wgrad_kernel<DT, LMAX, CPT, GR>);
  p.slabs = static_cast<int>((C / CPT + 63) / 64);
  const int64_t want = static_cast<int64_t>(num_cus()) * per_cu / p.slabs;
  p.nbx = std::max<int64_t>(1, std::min<int64_t>(want, (ncells + WC - 1) / WC));
}

WgradPlan wgrad_plan(int dt, int64_t ncells, int G, int64_t C, int L, int blocks_per_cu = 2) {
  WgradPlan p{};
  if (ncells > 0 && L <= kCellMaxDepth && fits32(ncells * kK * C * esize(dt))) {
    p.cell = true;
    dispatch_dtype(dt, [&](auto d) {
      constexpr int DT = decltype(d)::value;
      if (L <= 1) cell_wgrad_plan_l<DT, 1>(p, ncells, G, C);
      else if (L <= 2) cell_wgrad_plan_l<DT, 2>(p, ncells, G, C);
      else if (L <= 4) cell_wgrad_plan_l<DT, 4>(p, ncells, G, C);
      else if (L <= 8) cell_wgrad_plan_l<DT, 8>(p, ncells, G, C);
      else if (L <= 12) cell_wgrad_plan_l<DT, 12>(p, ncells, G, C);
      else if (L <= 16) cell_wgrad_plan_l<DT, 16>(p, ncells, G, C);
      else cell_wgrad_plan_l<DT, 24>(p, ncells, G, C);
    });
    return p;
  }
  int cpt = 4;
  wgrad_shape(L, p.tpt, cpt);
  const int qs = kBlock / (kK / p.tpt);
  p.slabs = static_cast<int>((C / cpt + qs - 1) / qs);
  p.cpb = cells_per_block(ncells, p.slabs, blocks_per_cu);
  p.nbx = ncells > 0 ? (ncells + p.cpb - 1) / p.cpb : 0;
  return p;
}

// Read blocks per CU (one: measured best for the 16-tap vector loads).
constexpr int kReadBlocksPerCU = 1;

template <int DT, int WDT, typename Off>
void launch_read(const void* x, const void* w, void* z, int64_t ncells, int G, int C, bool vec8, hipStream_t st) {
  const int vec = vec8 ? 8 : 4;
  const int ncv = C / vec;
  const int ncv_blk = std::min(ncv, kBlock);
  const int cpi = kBlock / ncv_blk;
  const int gy = (ncv + ncv_blk - 1) / ncv_blk;
  const int64_t step = grid_step_cells(static_cast<int64_t>(num_cus()) * kReadBlocksPerCU * cpi / gy, ncells, G, cpi);
  const dim3 grid(static_cast<unsigned>(step / cpi), gy);
  const dim3 block(ncv_blk * cpi);
  if constexpr (DT != LTHC_F32) {
    if (vec8) {
      read_fwd_kernel<DT, WDT, 8, Off><<<grid, block, 0, st>>>(x, w, z, ncells, G, C, ncv_blk, cpi);
      return;
    }
  }
  read_fwd_kernel<DT, WDT, 4, Off><<<grid, block, 0, st>>>(x, w, z, ncells, G, C, ncv_blk, cpi);
}

// Thread shapes (taps x channels per thread) of the register-resident weight
// kernels, per depth bucket: the weights (LMAX x TPT x CPT fp32) plus one
// cell's loads must fit in 256 VGPRs with two or more waves per SIMD.
template <int LMAX>
struct CellShape {
  static constexpr int TPT = LMAX <= 8 ? 4 : (LMAX <= 16 ? 4 : (LMAX <= 32 ? 2 : 1));
  static constexpr int CPT = LMAX <= 8 ? 4 : 2;
};
void wgrad_shape(int L, int& tpt, int& cpt) {
#define LTHC_WS(LM)              \
  {                              \
    tpt = CellShape<LM>::TPT;    \
    cpt = CellShape<LM>::CPT;    \
    return;                      \
  }
  if (L <= 1) LTHC_WS(1);
  if (L <= 2) LTHC_WS(2);
  if (L <= 4) LTHC_WS(4);
  if (L <= 8) LTHC_WS(8);
  if (L <= 12) LTHC_WS(12);
  if (L <= 16) LTHC_WS(16);
  if (L <= 24) LTHC_WS(24);
  if (L <= 32) LTHC_WS(32);
  LTHC_WS(48);
#undef LTHC_WS
}

constexpr int kMatBlocksPerCU = 6;

template <int DT, int WDT, int LMAX, int TPT, int CPT, bool HAS_BASE, bool EXACT, bool NT, typename Off>
void launch_mat_t(const void* base, const PtrPack& dz, const PtrPack& beta, void* out, int L, int64_t ncells, int G,
                  int C, int blocks_per_cu, hipStream_t st) {
  constexpr int QS = kBlock / (kK / TPT);
  const int slabs = (C / CPT + QS - 1) / QS;
  const int64_t cpb = cells_per_block(ncells, slabs, blocks_per_cu);
  const dim3 grid(static_cast<unsigned>((ncells + cpb - 1) / cpb), slabs);
  materialise_kernel<DT, WDT, LMAX, TPT, CPT, HAS_BASE, EXACT, NT, Off>
      <<<grid, kBlock, 0, st>>>(base, dz, beta, out, L, ncells, G, C, cpb);
}

template <int DT, int WDT, int LMAX>
void launch_mat_l(const void* base, const PtrPack& dz, const PtrPack& beta, void* out, int L, int64_t ncells, int G,
                  int C, bool off32, hipStream_t st) {
  constexpr int TPT = CellShape<LMAX>::TPT, CPT = CellShape<LMAX>::CPT;
  if (!off32)  // tensors of 4 GiB and more: 64-bit offsets, any depth in the bucket
    launch_mat_t<DT, WDT, LMAX, TPT, CPT, true, false, true, int64_t>(base, dz, beta, out, L, ncells, G, C, kMatBlocksPerCU, st);
  else if (L == LMAX)
    launch_mat_t<DT, WDT, LMAX, TPT, CPT, true, true, true, uint32_t>(base, dz, beta, out, L, ncells, G, C, kMatBlocksPerCU, st);
  else
    launch_mat_t<DT, WDT, LMAX, TPT, CPT, true, false, true, uint32_t>(base, dz, beta, out, L, ncells, G, C, kMatBlocksPerCU, st);
}

template <int DT, int WDT, int LMAX, bool HAS_BASE, bool EXACT>
void launch_cell_mat(const void* base, const PtrPack& dz, const PtrPack& beta, void* out, int L, int64_t ncells, int G,
                     int C, hipStream_t st) {
  constexpr int CPT = CellMatShape<DT, LMAX>::CPT, GR = CellMatShape<DT, LMAX>::GR;
  const auto kernel = cell_mat_kernel<DT, WDT, LMAX, CPT, GR, HAS_BASE, EXACT>;
  static const int per_cu = resident_blocks(kernel);
  const int slabs = (C / CPT + kBlock / GR - 1) / (kBlock / GR);
  const int64_t per = grid_cells(static_cast<int64_t>(num_cus()) * per_cu / slabs, ncells, 1);
  kernel<<<dim3(static_cast<unsigned>(per), slabs), kBlock, 0, st>>>(base, dz, beta, out, L,
                                                                    static_cast<uint32_t>(ncells), G, C);
}

// Layers whose weights the deep materialisation keeps in VGPRs: 242 VGPRs at depth 24, two wavefronts per SIMD (with
// 12 layers it spilled; 6 and 8 measured slower on MI355X).
constexpr int kDeepRegLayers = 10;
constexpr int kDeepRegLayers2 = 4;  // two cells per wavefront and step

template <int DT, int WDT, int LMAX, bool EXACT>
void launch_cell_mat_deep(const void* base, const PtrPack& dz, const PtrPack& beta, void* out, int L, int64_t ncells,
                          int G, int C, hipStream_t st) {
  PtrPack dp = dz, bp = beta;  // padding layers: layer 0's rows (contributing a selected 0)
  for (int l = L; l < LMAX; ++l) {
    dp.p[l] = dz.p[0];
    bp.p[l] = beta.p[0];
  }
  const int slabs = (C + 63) / 64;
  auto run = [&](auto nc, auto lv) {
    constexpr int NC = decltype(nc)::value, LV = decltype(lv)::value;
    const auto kernel = cell_mat_deep_kernel<DT, WDT, LMAX, LV, NC, EXACT>;
    static const int per_cu = resident_blocks(kernel);
    const int64_t per = grid_cells(static_cast<int64_t>(num_cus()) * per_cu * 4 * NC / slabs, ncells, 4 * NC);
    kernel<<<dim3(static_cast<unsigned>(per / (4 * NC)), slabs), kBlock, 0, st>>>(base, dp, bp, out, L,
                                                                                 static_cast<uint32_t>(ncells), G, C);
  };
  if (G % 8 == 0) run(IC<2>{}, IC<kDeepRegLayers2>{});  // two cells per wavefront and step
  else run(IC<1>{}, IC<kDeepRegLayers>{});
}

template <int DT, int WDT, int LMAX>
void launch_cell_mat_l(const void* base, const PtrPack& dz, const PtrPack& beta, void* out, int L, int64_t ncells,
                       int G, int C, hipStream_t st) {
  // depths 17-24 with a base: the deep kernel, which requests each dz run once per cell (5-6 % faster at depth 24
  // on configuration 5's shape, bitwise equal).  At depth 16 it was faster at C = 768 and slower at C = 1024 (where
  // cell_mat_kernel's two tap groups run three wavefronts per SIMD), and without a base it spilled.
  if constexpr (LMAX == 24) {
    if (base != nullptr) {
      if (L == LMAX) launch_cell_mat_deep<DT, WDT, LMAX, true>(base, dz, beta, out, L, ncells, G, C, st);
      else launch_cell_mat_deep<DT, WDT, LMAX, false>(base, dz, beta, out, L, ncells, G, C, st);
      return;
    }
  }
  if (base == nullptr) {  // the sum of writes alone (the adjoint of a multi-weight read)
    if (L == LMAX) launch_cell_mat<DT, WDT, LMAX, false, true>(base, dz, beta, out, L, ncells, G, C, st);
    else launch_cell_mat<DT, WDT, LMAX, false, false>(base, dz, beta, out, L, ncells, G, C, st);
  } else if (L == LMAX) {
    launch_cell_mat<DT, WDT, LMAX, true, true>(base, dz, beta, out, L, ncells, G, C, st);
  } else {
    launch_cell_mat<DT, WDT, LMAX, true, false>(base, dz, beta, out, L, ncells, G, C, st);
  }
}

template <int DT, int WDT>
void launch_materialise(const void* base, const PtrPack& dz, const PtrPack& beta, void* out, int L, int64_t ncells,
                        int G, int C, hipStream_t st) {
  const bool off32 = fits32(ncells * kK * C * Fmt<DT>::bytes);
  if (base == nullptr && !off32) {  // the plain write, tensors of 4 GiB and more: one layer (validated by the caller)
    launch_mat_t<DT, WDT, 1, 4, 4, false, true, true, int64_t>(base, dz, beta, out, 1, ncells, G, C, kMatBlocksPerCU, st);
    return;
  }
  if (off32 && L <= kCellMaxDepth) {  // whole-cell kernel: weights of every tap in VGPRs
    if (L <= 1) launch_cell_mat_l<DT, WDT, 1>(base, dz, beta, out, L, ncells, G, C, st);
    else if (L <= 2) launch_cell_mat_l<DT, WDT, 2>(base, dz, beta, out, L, ncells, G, C, st);
    else if (L <= 4) launch_cell_mat_l<DT, WDT, 4>(base, dz, beta, out, L, ncells, G, C, st);
    else if (L <= 8) launch_cell_mat_l<DT, WDT, 8>(base, dz, beta, out, L, ncells, G, C, st);
    else if (L <= 12) launch_cell_mat_l<DT, WDT, 12>(base, dz, beta, out, L, ncells, G, C, st);
    else if (L <= 16) launch_cell_mat_l<DT, WDT, 16>(base, dz, beta, out, L, ncells, G, C, st);
    else launch_cell_mat_l<DT, WDT, 24>(base, dz, beta, out, L, ncells, G, C, st);
    return;
  }
  if (L <= 1) launch_mat_l<DT, WDT, 1>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else if (L <= 2) launch_mat_l<DT, WDT, 2>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else if (L <= 4) launch_mat_l<DT, WDT, 4>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else if (L <= 8) launch_mat_l<DT, WDT, 8>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else if (L <= 12) launch_mat_l<DT, WDT, 12>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else if (L <= 16) launch_mat_l<DT, WDT, 16>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else if (L <= 24) launch_mat_l<DT, WDT, 24>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else if (L <= 32) launch_mat_l<DT, WDT, 32>(base, dz, beta, out, L, ncells, G, C, off32, st);
  else launch_mat_l<DT, WDT, 48>(base, dz, beta, out, L, ncells, G, C, off32, st);
}

template <int DT, int LMAX, int TPT, int CPT, bool NT, typename Off>
void launch_wgrad_t(const void* high, const PtrPack& low, float* partial, int L, int64_t ncells, int G, int C,
                    const WgradPlan& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.nbx), p.slabs);
  wgrad_partial_kernel<DT, LMAX, TPT, CPT, NT, Off><<<grid, kBlock, 0, st>>>(high, low, partial, L, ncells, G, C, p.cpb);
}

template <int DT, int LMAX>
void launch_cell_wgrad(const void* high, const PtrPack& low, float* partial, int L, int64_t ncells, int G, int C,
                       const WgradPlan& p, hipStream_t st) {
  constexpr int CPT = CellMatShape<DT, LMAX>::CPT, GR = CellMatShape<DT, LMAX>::GR;
  cell_wgrad_kernel<DT, LMAX, CPT, GR><<<dim3(static_cast<unsigned>(p.nbx), p.slabs), kBlock, 0, st>>>(
      high, low, partial, L, static_cast<uint32_t>(ncells), G, C);
}

template <int DT, typename Off>
void launch_wgrad(const void* high, const PtrPack& low, float* partial, int L, int64_t ncells, int G, int C,
                  const WgradPlan& p, hipStream_t st) {
  if constexpr (std::is_same_v<Off, uint32_t>) {
    if (p.cell) {
      if (L <= 1) launch_cell_wgrad<DT, 1>(high, low, partial, L, ncells, G, C, p, st);
      else if (L <= 2) launch_cell_wgrad<DT, 2>(high, low, partial, L, ncells, G, C, p, st);
      else if (L <= 4) launch_cell_wgrad<DT, 4>(high, low, partial, L, ncells, G, C, p, st);
      else if (L <= 8) launch_cell_wgrad<DT, 8>(high, low, partial, L, ncells, G, C, p, st);
      else if (L <= 12) launch_cell_wgrad<DT, 12>(high, low, partial, L, ncells, G, C, p, st);
      else if (L <= 16) launch_cell_wgrad<DT, 16>(high, low, partial, L, ncells, G, C, p, st);
      else launch_cell_wgrad<DT, 24>(high, low, partial, L, ncells, G, C, p, st);
      return;
    }
  }
#define LTHC_WG(LM) \
  launch_wgrad_t<DT, LM, CellShape<LM>::TPT, CellShape<LM>::CPT, true, Off>(high, low, partial, L, ncells, G, C, p, st)
  if (L <= 1) LTHC_WG(1);
  else if (L <= 2) LTHC_WG(2);
  else if (L <= 4) LTHC_WG(4);
  else if (L <= 8) LTHC_WG(8);
  else if (L <= 12) LTHC_WG(12);
  else if (L <= 16) LTHC_WG(16);
  else if (L <= 24) LTHC_WG(24);
  else if (L <= 32) LTHC_WG(32);
  else LTHC_WG(48);
#undef LTHC_WG
}

template <int DT, int WDT, int LC, typename Off>
void launch_read_multi_t(const void* g, const PtrPack& w, const PtrPack& out, int L, int64_t ncells, int G, int C,
                         hipStream_t st) {
  const int nlg = (L + LC - 1) / LC;
  const int qs = std::max(16, (kBlock / nlg) / 16 * 16);  // qs * nlg <= 256 for nlg <= 16
  const int slabs = (C / 4 + qs - 1) / qs;
  const int64_t cpb = cells_per_block(ncells, slabs, 8);
  const dim3 grid(static_cast<unsigned>((ncells + cpb - 1) / cpb), slabs);
  read_multi_kernel<DT, WDT, LC, Off><<<grid, qs * nlg, 0, st>>>(g, w, out, L, qs, ncells, G, C, cpb);
}

template <int DT, int WDT, int LMAX>
void launch_cell_read_multi(const void* g, const PtrPack& w, const PtrPack& out, int L, int64_t ncells, int G, int C,
                            hipStream_t st) {
  constexpr int CPT = CellMatShape<DT, LMAX>::CPT, GR = CellMatShape<DT, LMAX>::GR;
  const auto kernel = L == LMAX ? cell_read_multi_kernel<DT, WDT, LMAX, CPT, GR, true>
                                : cell_read_multi_kernel<DT, WDT, LMAX, CPT, GR, false>;
  static const int per_cu = resident_blocks(cell_read_multi_kernel<DT, WDT, LMAX, CPT, GR, false>);
  const int slabs = (C / CPT + kBlock / GR - 1) / (kBlock / GR);
  const int64_t per = grid_cells(static_cast<int64_t>(num_cus()) * per_cu / slabs, ncells, 1);
  kernel<<<dim3(static_cast<unsigned>(per), slabs), kBlock, 0, st>>>(g, w, out, L, static_cast<uint32_t>(ncells), G, C);
}

template <int DT, int WDT, typename Off>
void launch_read_multi(const void* g, const PtrPack& w, const PtrPack& out, int L, int64_t ncells, int G, int C,
                       hipStream_t st) {
  if constexpr (std::is_same_v<Off, uint32_t>) {  // whole-cell kernel: every layer's weights in VGPRs
    if (L <= kCellMaxDepth) {
      if (L <= 1) launch_cell_read_multi<DT, WDT, 1>(g, w, out, L, ncells, G, C, st);
      else if (L <= 2) launch_cell_read_multi<DT, WDT, 2>(g, w, out, L, ncells, G, C, st);
      else if (L <= 4) launch_cell_read_multi<DT, WDT, 4>(g, w, out, L, ncells, G, C, st);
      else if (L <= 8) launch_cell_read_multi<DT, WDT, 8>(g, w, out, L, ncells, G, C, st);
      else if (L <= 12) launch_cell_read_multi<DT, WDT, 12>(g, w, out, L, ncells, G, C, st);
      else if (L <= 16) launch_cell_read_multi<DT, WDT, 16>(g, w, out, L, ncells, G, C, st);
      else launch_cell_read_multi<DT, WDT, 24>(g, w, out, L, ncells, G, C, st);
      return;
    }
  }
  // Two layers per thread keep 128 weights + loads + accumulators within 256
  // VGPRs; three per thread only where 16 groups of two are not enough.
  if (L == 1) launch_read_multi_t<DT, WDT, 1, Off>(g, w, out, L, ncells, G, C, st);
  else if (L <= 32) launch_read_multi_t<DT, WDT, 2, Off>(g, w, out, L, ncells, G, C, st);
  else launch_read_multi_t<DT, WDT, 3, Off>(g, w, out, L, ncells, G, C, st);
}

int fill_ptrs(const char* fn, PtrPack& pk, const void* const* src, int L, const char* name, int dt, bool act) {
  if (src == nullptr) return fail(LTHC_ERR_INVALID, fn, std::string(name) + " pointer array is NULL");
  for (int l = 0; l < L; ++l) {
    const std::string nm = std::string(name) + "[" + std::to_string(l) + "]";
    if (act) {
      if (int rc = check_act(fn, src[l], dt, nm.c_str())) return rc;
    } else {
      if (int rc = check_weight(fn, src[l], nm)) return rc;
    }
    pk.p[l] = src[l];
  }
  for (int l = L; l < LTHC_MAX_LAYERS; ++l) pk.p[l] = nullptr;
  return LTHC_OK;
}

int check_layers(const char* fn, int L) {
  if (L < 1) return fail(LTHC_ERR_INVALID, fn, "L must be >= 1");
  if (L > LTHC_MAX_LAYERS) return fail(LTHC_ERR_UNSUPPORTED, fn, "L exceeds LTHC_MAX_LAYERS");
  return LTHC_OK;
}

int check_pair(const char* fn, int x_dtype, int w_dtype) {
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (!supported_pair(x_dtype, w_dtype))
    return fail(LTHC_ERR_UNSUPPORTED, fn, "weights must be fp32 or have the activation dtype");
  return LTHC_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* lthc_last_error(void) { return g_last_error.c_str(); }

int lthc_abi_version(void) { return 3; }

int lthc_read_fwd(const void* x, int x_dtype, const void* alpha, int w_dtype, void* z, int64_t B, int64_t G, int64_t s,
                  int64_t C, void* stream) {
  static const char* fn = "lthc_read_fwd";
  g_last_error.clear();
  if (int rc = check_geom(fn, B, G, s, C)) return rc;
  if (int rc = check_pair(fn, x_dtype, w_dtype)) return rc;
  if (B == 0) return LTHC_OK;
  if (int rc = check_act(fn, x, x_dtype, "x")) return rc;
  if (int rc = check_act(fn, z, x_dtype, "z")) return rc;
  if (int rc = check_weight(fn, alpha, "alpha")) return rc;
  const int64_t ncells = B * G * G;
  const bool vec8 = x_dtype != LTHC_F32 && C % 8 == 0 && aligned(x, 16) && aligned(z, 16);
  const bool off32 = fits32(ncells * kK * C * esize(x_dtype));
  dispatch_pair(x_dtype, w_dtype, [&](auto d, auto wd) {
    dispatch_off(off32, [&](auto o) {
      launch_read<decltype(d)::value, decltype(wd)::value, typename decltype(o)::type>(
          x, alpha, z, ncells, static_cast<int>(G), static_cast<int>(C), vec8, static_cast<hipStream_t>(stream));
    });
  });
  return check_launch(fn);
}

int lthc_read_multi_fwd(const void* g, int x_dtype, const void* const* w, int w_dtype, void* const* out, int64_t B,
                        int64_t G, int64_t s, int64_t C, int L, void* stream) {
  static const char* fn = "lthc_read_multi_fwd";
  g_last_error.clear();
  if (int rc = check_geom(fn, B, G, s, C)) return rc;
  if (int rc = check_layers(fn, L)) return rc;
  if (int rc = check_pair(fn, x_dtype, w_dtype)) return rc;
  if (B == 0) return LTHC_OK;
  if (int rc = check_act(fn, g, x_dtype, "g")) return rc;
  PtrPack wp, op;
  if (int rc = fill_ptrs(fn, wp, w, L, "w", w_dtype, false)) return rc;
  if (int rc = fill_ptrs(fn, op, const_cast<const void* const*>(out), L, "out", x_dtype, true)) return rc;
  const int64_t ncells = B * G * G;
  const bool off32 = fits32(ncells * kK * C * esize(x_dtype));
  dispatch_pair(x_dtype, w_dtype, [&](auto d, auto wd) {
    dispatch_off(off32, [&](auto o) {
      launch_read_multi<decltype(d)::value, decltype(wd)::value, typename decltype(o)::type>(
          g, wp, op, L, ncells, static_cast<int>(G), static_cast<int>(C), static_cast<hipStream_t>(stream));
    });
  });
  return check_launch(fn);
}

int lthc_materialise_fwd(const void* base, const void* const* dz, int x_dtype, const void* const* beta, int w_dtype,
                         void* out, int64_t B, int64_t G, int64_t s, int64_t C, int L, void* stream) {
  static const char* fn = "lthc_materialise_fwd";
  g_last_error.clear();
  if (int rc = check_geom(fn, B, G, s, C)) return rc;
  if (int rc = check_layers(fn, L)) return rc;
  if (int rc = check_pair(fn, x_dtype, w_dtype)) return rc;
  if (base == nullptr && L != 1 && (L > kCellMaxDepth || !fits32(B * G * G * kK * C * esize(x_dtype))))
    return fail(LTHC_ERR_UNSUPPORTED, fn, "base == NULL is implemented for L == 1, or L <= 24 below 4 GiB");
  if (B == 0) return LTHC_OK;
  if (base != nullptr)
    if (int rc = check_act(fn, base, x_dtype, "base")) return rc;
  if (int rc = check_act(fn, out, x_dtype, "out")) return rc;
  PtrPack dp, bp;
  if (int rc = fill_ptrs(fn, dp, dz, L, "dz", x_dtype, true)) return rc;
  if (int rc = fill_ptrs(fn, bp, beta, L, "beta", w_dtype, false)) return rc;
  const int64_t ncells = B * G * G;
  dispatch_pair(x_dtype, w_dtype, [&](auto d, auto wd) {
    launch_materialise<decltype(d)::value, decltype(wd)::value>(base, dp, bp, out, L, ncells, static_cast<int>(G),
                                                                static_cast<int>(C), static_cast<hipStream_t>(stream));
  });
  return check_launch(fn);
}

size_t lthc_weight_grad_workspace_bytes(int64_t B, int64_t G, int64_t s, int64_t C, int L) {
  if (B <= 0 || G <= 0 || C <= 0 || L < 1 || s != kS || C % 4 != 0 || G > 4096 || C > (1 << 24)) return 0;
  if (B > (int64_t(1) << 40) / (G * G * kK * C)) return 0;
  // the plan depends on the activation dtype: return the largest over the dtypes
  int64_t nbx = 0;
  for (int dt : {LTHC_F32, LTHC_BF16, LTHC_F16}) nbx = std::max(nbx, wgrad_plan(dt, B * G * G, static_cast<int>(G), C, L).nbx);
  return static_cast<size_t>(nbx) * static_cast<size_t>(L) * static_cast<size_t>(C) * kK * sizeof(float);
}

int lthc_weight_grad(const void* high, const void* const* low, int x_dtype, float* gw, int64_t B, int64_t G, int64_t s,
                     int64_t C, int L, void* workspace, size_t workspace_bytes, void* stream) {
  static const char* fn = "lthc_weight_grad";
  g_last_error.clear();
  if (int rc = check_geom(fn, B, G, s, C)) return rc;
  if (int rc = check_layers(fn, L)) return rc;
  if (!valid_dtype(x_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (gw == nullptr) return fail(LTHC_ERR_INVALID, fn, "gw is NULL");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = static_cast<int64_t>(L) * C * kK;
  if (B == 0) {
    zero_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(gw, n);
    return check_launch(fn);
  }
  if (int rc = check_act(fn, high, x_dtype, "high")) return rc;
  PtrPack lp;
  if (int rc = fill_ptrs(fn, lp, low, L, "low", x_dtype, true)) return rc;
  const int64_t ncells = B * G * G;
  const WgradPlan p = wgrad_plan(x_dtype, ncells, static_cast<int>(G), C, L);
  const size_t need = static_cast<size_t>(p.nbx) * n * sizeof(float);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LTHC_ERR_INVALID, fn, "workspace smaller than lthc_weight_grad_workspace_bytes()");
  if (!aligned(workspace, 16)) return fail(LTHC_ERR_INVALID, fn, "workspace is not 16-byte aligned");
  float* partial = static_cast<float*>(workspace);
  const bool off32 = fits32(ncells * kK * C * esize(x_dtype));
  dispatch_dtype(x_dtype, [&](auto d) {
    dispatch_off(off32, [&](auto o) {
      launch_wgrad<decltype(d)::value, typename decltype(o)::type>(high, lp, partial, L, ncells, static_cast<int>(G),
                                                                   static_cast<int>(C), p, st);
    });
  });
  if (int rc = check_launch(fn)) return rc;
  launch_reduce(partial, static_cast<int>(p.nbx), n, gw, st);
  return check_launch(fn);
}

int lthc_gamma(const void* alpha, const void* const* beta, int w_dtype, void* gamma, int out_dtype, int64_t C,
               int64_t K, int L, void* stream) {
  static const char* fn = "lthc_gamma";
  g_last_error.clear();
  if (int rc = check_layers(fn, L)) return rc;
  if (C <= 0 || K <= 0 || K > 1024 || C > (1 << 24)) return fail(LTHC_ERR_INVALID, fn, "C or K out of range");
  if (!valid_dtype(w_dtype) || !valid_dtype(out_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (alpha == nullptr || gamma == nullptr) return fail(LTHC_ERR_INVALID, fn, "alpha or gamma is NULL");
  PtrPack bp;
  if (beta == nullptr) return fail(LTHC_ERR_INVALID, fn, "beta pointer array is NULL");
  for (int l = 0; l < L; ++l) {
    if (beta[l] == nullptr) return fail(LTHC_ERR_INVALID, fn, "beta[" + std::to_string(l) + "] is NULL");
    bp.p[l] = beta[l];
  }
  const int64_t n = static_cast<int64_t>(L) * C;
  const unsigned blocks = static_cast<unsigned>((n + 255) / 256);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  bool rows16 = K == kK && aligned(alpha, 16);
  for (int l = 0; l < L; ++l) rows16 = rows16 && aligned(beta[l], 16);
  if (rows16) {
    dispatch_dtype(w_dtype, [&](auto wd) {
      dispatch_dtype(out_dtype, [&](auto od) {
        gamma16_kernel<decltype(wd)::value, decltype(od)::value><<<blocks, 256, 0, st>>>(alpha, bp, gamma,
                                                                                         static_cast<int>(C), L);
      });
    });
    return check_launch(fn);
  }
  gamma_kernel<<<blocks, 256, 0, st>>>(alpha, bp, w_dtype, gamma, out_dtype, static_cast<int>(C), static_cast<int>(K), L);
  return check_launch(fn);
}

int lthc_gamma_rounded(const void* alpha, int a_dtype, const void* const* beta, int b_dtype, void* gamma,
                       int out_dtype, int64_t C, int64_t K, int L, void* stream) {
  static const char* fn = "lthc_gamma_rounded";
  g_last_error.clear();
  if (int rc = check_layers(fn, L)) return rc;
  if (C <= 0 || K <= 0 || K > 1024 || C > (1 << 24)) return fail(LTHC_ERR_INVALID, fn, "C or K out of range");
  if (!valid_dtype(a_dtype) || !valid_dtype(b_dtype) || !valid_dtype(out_dtype))
    return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (alpha == nullptr || gamma == nullptr || beta == nullptr) return fail(LTHC_ERR_INVALID, fn, "a NULL pointer");
  PtrPack bp;
  for (int l = 0; l < L; ++l) {
    if (beta[l] == nullptr) return fail(LTHC_ERR_INVALID, fn, "beta[" + std::to_string(l) + "] is NULL");
    bp.p[l] = beta[l];
  }
  const int64_t n = static_cast<int64_t>(L) * C;
  const unsigned blocks = static_cast<unsigned>((n + 255) / 256);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  bool rows16 = K == kK && aligned(alpha, 16);
  for (int l = 0; l < L; ++l) rows16 = rows16 && aligned(beta[l], 16);
  if (rows16) {
    dispatch_dtype(out_dtype, [&](auto d) {
      dispatch_dtype(a_dtype, [&](auto ad) {
        dispatch_dtype(b_dtype, [&](auto bd) {
          gamma16_rounded_kernel<decltype(d)::value, decltype(ad)::value, decltype(bd)::value>
              <<<blocks, 256, 0, st>>>(alpha, bp, gamma, static_cast<int>(C), L);
        });
      });
    });
    return check_launch(fn);
  }
  dispatch_dtype(out_dtype, [&](auto d) {
    gamma_rounded_kernel<decltype(d)::value><<<blocks, 256, 0, st>>>(alpha, a_dtype, bp, b_dtype, gamma,
                                                                     static_cast<int>(C), static_cast<int>(K), L);
  });
  return check_launch(fn);
}

int lthc_gamma_rounded_bwd(const void* grad, const void* alpha, int a_dtype, const void* const* beta, int b_dtype,
                           void* galpha, void* const* gbeta, int out_dtype, int64_t C, int64_t K, int L,
                           void* stream) {
  static const char* fn = "lthc_gamma_rounded_bwd";
  g_last_error.clear();
  if (int rc = check_layers(fn, L)) return rc;
  if (C <= 0 || K <= 0 || K > 1024 || C > (1 << 24)) return fail(LTHC_ERR_INVALID, fn, "C or K out of range");
  if (!valid_dtype(a_dtype) || !valid_dtype(b_dtype) || !valid_dtype(out_dtype))
    return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (grad == nullptr || alpha == nullptr || beta == nullptr) return fail(LTHC_ERR_INVALID, fn, "a NULL pointer");
  PtrPack bp, gp;
  for (int l = 0; l < L; ++l) {
    if (beta[l] == nullptr) return fail(LTHC_ERR_INVALID, fn, "beta[" + std::to_string(l) + "] is NULL");
    bp.p[l] = beta[l];
    gp.p[l] = gbeta == nullptr ? nullptr : gbeta[l];
  }
  const int64_t n = C * K;
  const int64_t nb_beta = gbeta == nullptr ? 0 : (n * L + 255) / 256;
  const int64_t nb_alpha = galpha == nullptr ? 0 : (n + 255) / 256;
  if (nb_beta + nb_alpha == 0) return LTHC_OK;
  dispatch_dtype(out_dtype, [&](auto d) {
    dispatch_dtype(b_dtype, [&](auto bd) {
      constexpr int ODT = decltype(d)::value, BDT = decltype(bd)::value;
      const auto kernel = L <= 12   ? gamma_rounded_bwd_kernel<ODT, BDT, 12>
                          : L <= 24 ? gamma_rounded_bwd_kernel<ODT, BDT, 24>
                                    : gamma_rounded_bwd_kernel<ODT, BDT, LTHC_MAX_LAYERS>;
      kernel<<<static_cast<unsigned>(nb_beta + nb_alpha), 256, 0, static_cast<hipStream_t>(stream)>>>(
          grad, alpha, a_dtype, bp, galpha, gp, static_cast<int>(C), static_cast<int>(K), L,
          static_cast<int>(nb_beta));
    });
  });
  return check_launch(fn);
}

int lthc_recur_fwd(const void* z, const void* dz, int x_dtype, const void* gamma, int g_dtype, void* z_next,
                   int64_t rows, int64_t C, void* stream) {
  static const char* fn = "lthc_recur_fwd";
  g_last_error.clear();
  if (rows < 0 || C <= 0 || C % 4 != 0 || C > (1 << 24)) return fail(LTHC_ERR_INVALID, fn, "rows >= 0 and C > 0, C % 4 == 0 required");
  if (!valid_dtype(x_dtype) || !valid_dtype(g_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (rows == 0) return LTHC_OK;
  if (int rc = check_act(fn, z, x_dtype, "z")) return rc;
  if (int rc = check_act(fn, dz, x_dtype, "dz")) return rc;
  if (int rc = check_act(fn, z_next, x_dtype, "z_next")) return rc;
  if (gamma == nullptr) return fail(LTHC_ERR_INVALID, fn, "gamma is NULL");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool off32 = fits32(rows * C * esize(x_dtype));
  const int64_t vec = 16 / esize(x_dtype);
  if (off32 && C % vec == 0 && aligned(z, 16) && aligned(dz, 16) && aligned(z_next, 16) &&
      aligned(gamma, 16)) {
    const uint32_t nvec = static_cast<uint32_t>(rows * C / vec);
    dispatch_dtype(x_dtype, [&](auto d) {
      dispatch_dtype(g_dtype, [&](auto gd) {
        recur_fwd_flat_kernel<decltype(d)::value, decltype(gd)::value><<<(nvec + 255) / 256, 256, 0, st>>>(
            z, dz, gamma, z_next, nvec, static_cast<uint32_t>(C / vec));
      });
    });
    return check_launch(fn);
  }
  const int64_t chunks = (rows + 4 * kRU - 1) / (4 * kRU);
  const dim3 grid(static_cast<unsigned>((C / 4 + 63) / 64), static_cast<unsigned>(std::min(chunks, kRecurChunks)));
  dispatch_dtype(x_dtype, [&](auto d) {
    dispatch_off(off32, [&](auto o) {
      recur_fwd_kernel<decltype(d)::value, typename decltype(o)::type>
          <<<grid, 256, 0, st>>>(z, dz, gamma, g_dtype, z_next, rows, static_cast<int>(C));
    });
  });
  return check_launch(fn);
}

size_t lthc_recur_bwd_workspace_bytes(int64_t rows, int64_t C) {
  if (rows <= 0 || C <= 0) return 0;
  return static_cast<size_t>(recur_bwd_blocks_y(rows) * C) * sizeof(float);
}

int lthc_recur_bwd(const void* g, const void* dz, const void* gdz_add, int x_dtype, const void* gamma, int g_dtype,
                   void* gdz, float* ggamma, int64_t rows, int64_t C, void* workspace, size_t workspace_bytes,
                   void* stream) {
  static const char* fn = "lthc_recur_bwd";
  g_last_error.clear();
  if (rows < 0 || C <= 0 || C % 4 != 0 || C > (1 << 24)) return fail(LTHC_ERR_INVALID, fn, "rows >= 0 and C > 0, C % 4 == 0 required");
  if (!valid_dtype(x_dtype) || !valid_dtype(g_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (ggamma == nullptr || gamma == nullptr) return fail(LTHC_ERR_INVALID, fn, "gamma or ggamma is NULL");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0) {
    zero_kernel<<<static_cast<unsigned>((C + 255) / 256), 256, 0, st>>>(ggamma, C);
    return check_launch(fn);
  }
  if (int rc = check_act(fn, g, x_dtype, "g")) return rc;
  if (int rc = check_act(fn, dz, x_dtype, "dz")) return rc;
  if (int rc = check_act(fn, gdz, x_dtype, "gdz")) return rc;
  if (gdz_add != nullptr)
    if (int rc = check_act(fn, gdz_add, x_dtype, "gdz_add")) return rc;
  const size_t need = lthc_recur_bwd_workspace_bytes(rows, C);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LTHC_ERR_INVALID, fn, "workspace smaller than lthc_recur_bwd_workspace_bytes()");
  if (!aligned(workspace, 16)) return fail(LTHC_ERR_INVALID, fn, "workspace is not 16-byte aligned");
  const int64_t by = recur_bwd_blocks_y(rows);
  const dim3 grid(static_cast<unsigned>((C / 4 + 63) / 64), static_cast<unsigned>(by));
  float* partial = static_cast<float*>(workspace);
  const bool off32 = fits32(rows * C * esize(x_dtype));
  dispatch_dtype(x_dtype, [&](auto d) {
    dispatch_off(off32, [&](auto o) {
      if (gdz_add != nullptr)
        recur_bwd_kernel<decltype(d)::value, typename decltype(o)::type, true>
            <<<grid, 256, 0, st>>>(g, dz, gdz_add, gamma, g_dtype, gdz, partial, rows, static_cast<int>(C));
      else
        recur_bwd_kernel<decltype(d)::value, typename decltype(o)::type, false>
            <<<grid, 256, 0, st>>>(g, dz, nullptr, gamma, g_dtype, gdz, partial, rows, static_cast<int>(C));
    });
  });
  if (int rc = check_launch(fn)) return rc;
  launch_reduce(partial, static_cast<int>(by), C, ggamma, st);
  return check_launch(fn);
}

int lthc_recur_bwd_sum(const void* g, const void* g_branch, const void* dz, const void* gdz_add, int x_dtype,
                       const void* gamma, int g_dtype, void* g_sum, void* gdz, void* ggamma, int gg_dtype,
                       int64_t rows, int64_t C, void* workspace, size_t workspace_bytes, void* stream) {
  static const char* fn = "lthc_recur_bwd_sum";
  g_last_error.clear();
  if (rows < 0 || C <= 0 || C % 4 != 0 || C > (1 << 24)) return fail(LTHC_ERR_INVALID, fn, "rows >= 0 and C > 0, C % 4 == 0 required");
  if (!valid_dtype(x_dtype) || !valid_dtype(g_dtype) || !valid_dtype(gg_dtype))
    return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (ggamma == nullptr || gamma == nullptr) return fail(LTHC_ERR_INVALID, fn, "gamma or ggamma is NULL");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0) {
    launch_reduce(nullptr, 0, C, ggamma, st, gg_dtype);  // no parts: zeros
    return check_launch(fn);
  }
  if (int rc = check_act(fn, g, x_dtype, "g")) return rc;
  if (int rc = check_act(fn, g_branch, x_dtype, "g_branch")) return rc;
  if (int rc = check_act(fn, dz, x_dtype, "dz")) return rc;
  if (int rc = check_act(fn, g_sum, x_dtype, "g_sum")) return rc;
  if (int rc = check_act(fn, gdz, x_dtype, "gdz")) return rc;
  if (gdz_add != nullptr)
    if (int rc = check_act(fn, gdz_add, x_dtype, "gdz_add")) return rc;
  const size_t need = lthc_recur_bwd_workspace_bytes(rows, C);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LTHC_ERR_INVALID, fn, "workspace smaller than lthc_recur_bwd_workspace_bytes()");
  if (!aligned(workspace, 16)) return fail(LTHC_ERR_INVALID, fn, "workspace is not 16-byte aligned");
  const int64_t by = recur_bwd_blocks_y(rows);
  const dim3 grid(static_cast<unsigned>((C / 4 + 63) / 64), static_cast<unsigned>(by));
  float* partial = static_cast<float*>(workspace);
  const bool off32 = fits32(rows * C * esize(x_dtype));
  dispatch_dtype(x_dtype, [&](auto d) {
    dispatch_off(off32, [&](auto o) {
      if (gdz_add != nullptr)
        recur_bwd_kernel<decltype(d)::value, typename decltype(o)::type, true, true><<<grid, 256, 0, st>>>(
            g, dz, gdz_add, gamma, g_dtype, gdz, partial, rows, static_cast<int>(C), g_branch, g_sum);
      else
        recur_bwd_kernel<decltype(d)::value, typename decltype(o)::type, false, true><<<grid, 256, 0, st>>>(
            g, dz, nullptr, gamma, g_dtype, gdz, partial, rows, static_cast<int>(C), g_branch, g_sum);
    });
  });
  if (int rc = check_launch(fn)) return rc;
  launch_reduce(partial, static_cast<int>(by), C, ggamma, st, gg_dtype);
  return check_launch(fn);
}

}  // extern "C"

// Final-layer RMSNorm + modulate of the decoder input (the materialisation's consumer).
#include "norm_modulate.inc"

// Workspace accumulation of the non-shared (triangular lazy) interface.
#include "ws_accumulate.inc"
#include "branch_ops.inc"
// Fused q/k RMSNorm + RoPE and attention of the branch (matrix cores).
#include "attention.inc"
// The decoder head (norm + modulate + linear + unpatchify) on the matrix cores.
#include "decoder.inc"
// One-launch dtype conversion of many weights (autocast's per-forward casts).
#include "cast_many.inc"
// LDS-staged backward tiles: the materialise backward and the single-pass interface backward.
#include "bwd_tile.inc"

#include "mat_bwd_mfma.inc"
// Fused materialise backward (gdZ and gbeta from one pass over G).
#include "materialise_bwd.inc"
// Whole-interface entry points: recurrence prefix, read backward, interface forward / backward.
#include "interface.inc"
// The materialise backward without a caller workspace (a file-scope scratch array per GPU).
#include "noalloc.inc"
// The materialisation with the decoder front in its epilogue (no-grad forwards).
#include "mat_decoder.inc"
