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
// moved.  Lanes of a wavefront always run along the channel axis so that a
// wavefront load covers one contiguous 512 B .. 1 KiB span of a tap; the
// per-channel weights a thread needs are loaded into VGPRs once per block
// and reused for every cell the block visits.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <cstdio>
#include <string>

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

template <int DT>
struct Fmt;
template <>
struct Fmt<LTHC_F32> {
  static constexpr int bytes = 4;
};
template <>
struct Fmt<LTHC_BF16> {
  static constexpr int bytes = 2;
};
template <>
struct Fmt<LTHC_F16> {
  static constexpr int bytes = 2;
};

template <int DT>
LTHC_DEV void unpack2(uint32_t w, float& a, float& b);
template <>
LTHC_DEV void unpack2<LTHC_BF16>(uint32_t w, float& a, float& b) {
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}
template <>
LTHC_DEV void unpack2<LTHC_F16>(uint32_t w, float& a, float& b) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, w);
  a = static_cast<float>(h.x);
  b = static_cast<float>(h.y);
}

// Round-to-nearest-even narrowing (v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
template <int DT>
LTHC_DEV uint32_t pack2(float a, float b);
template <>
LTHC_DEV uint32_t pack2<LTHC_BF16>(float a, float b) {
  const bf16x2_t r = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, r);
}
template <>
LTHC_DEV uint32_t pack2<LTHC_F16>(float a, float b) {
  const f16x2_t r = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(uint32_t, r);
}

// N consecutive elements starting at element index i, widened to fp32.
template <int DT, int N>
LTHC_DEV void load_vec(const void* __restrict__ p, int64_t i, float (&v)[N]) {
  static_assert(N == 4 || N == 8, "vector width");
  if constexpr (DT == LTHC_F32) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const float4 r = q[j];
      v[4 * j + 0] = r.x;
      v[4 * j + 1] = r.y;
      v[4 * j + 2] = r.z;
      v[4 * j + 3] = r.w;
    }
  } else {
    const uint16_t* q = static_cast<const uint16_t*>(p) + i;
    if constexpr (N == 4) {
      const uint2 r = *reinterpret_cast<const uint2*>(q);
      unpack2<DT>(r.x, v[0], v[1]);
      unpack2<DT>(r.y, v[2], v[3]);
    } else {
      const uint4 r = *reinterpret_cast<const uint4*>(q);
      unpack2<DT>(r.x, v[0], v[1]);
      unpack2<DT>(r.y, v[2], v[3]);
      unpack2<DT>(r.z, v[4], v[5]);
      unpack2<DT>(r.w, v[6], v[7]);
    }
  }
}

template <int DT, int N>
LTHC_DEV void store_vec(void* __restrict__ p, int64_t i, const float (&v)[N]) {
  static_assert(N == 4 || N == 8, "vector width");
  if constexpr (DT == LTHC_F32) {
    float4* q = reinterpret_cast<float4*>(static_cast<float*>(p) + i);
#pragma unroll
    for (int j = 0; j < N / 4; ++j) q[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
  } else {
    uint16_t* q = static_cast<uint16_t*>(p) + i;
    if constexpr (N == 4) {
      *reinterpret_cast<uint2*>(q) = make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
    } else {
      *reinterpret_cast<uint4*>(q) = make_uint4(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]),
                                                pack2<DT>(v[4], v[5]), pack2<DT>(v[6], v[7]));
    }
  }
}

// One weight element of a runtime dtype, widened to fp32.
LTHC_DEV float load_w(const void* __restrict__ p, int dt, int64_t i) {
  if (dt == LTHC_F32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  if (dt == LTHC_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
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

// Offset of tap (sy, sx0) of cell `cell` at channel c0 in an NHWC tensor.
LTHC_DEV int64_t tap_offset(int64_t cell, int G, int C, int sy, int sx0, int c0) {
  const int M = G * G;
  const int H = G * kS;
  const int64_t b = cell / M;
  const int m = static_cast<int>(cell - b * M);
  const int gy = m / G;
  const int gx = m - gy * G;
  return ((b * H + gy * kS + sy) * H + gx * kS + sx0) * static_cast<int64_t>(C) + c0;
}

// ---------------------------------------------------------------------------
// READ: z[cell, c] = sum_k alpha[c,k] x[cell, k, c]
// Thread = VEC channels of one cell, all 16 taps; alpha for those channels
// lives in VGPRs.  Block = cpi cells x ncv_blk channel vectors.
// ---------------------------------------------------------------------------
template <int DT, int VEC>
__global__ __launch_bounds__(kBlock) void read_fwd_kernel(const void* __restrict__ x, const void* __restrict__ w,
                                                          int wdt, void* __restrict__ z, int64_t ncells, int G,
                                                          int C, int ncv_blk, int cpi, int64_t cpb) {
  const int t = threadIdx.x;
  const int ci = t / ncv_blk;
  const int c0 = (blockIdx.y * ncv_blk + (t - ci * ncv_blk)) * VEC;
  if (ci >= cpi || c0 >= C) return;
  float a[kK][VEC];
#pragma unroll
  for (int k = 0; k < kK; ++k)
#pragma unroll
    for (int v = 0; v < VEC; ++v) a[k][v] = load_w(w, wdt, static_cast<int64_t>(c0 + v) * kK + k);

  const int64_t row = static_cast<int64_t>(G) * kS * C;  // one high-res row
  const int64_t cb = static_cast<int64_t>(blockIdx.x) * cpb;
  const int64_t ce = std::min(ncells, cb + cpb);
  for (int64_t cell = cb + ci; cell < ce; cell += cpi) {
    const int64_t o = tap_offset(cell, G, C, 0, 0, c0);
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      float xv[VEC];
      load_vec<DT, VEC>(x, o + (k / kS) * row + (k % kS) * C, xv);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = fmaf(xv[v], a[k][v], acc[v]);
    }
    store_vec<DT, VEC>(z, cell * C + c0, acc);
  }
}

// ---------------------------------------------------------------------------
// MATERIALISE / WRITE: out[cell,k,c] = base[cell,k,c] + sum_l beta_l[c,k] dz_l[cell,c]
// Thread = 4 channels x TPT taps of one tap row; its LMAX x TPT x 4 write
// weights stay in VGPRs.  Block = 256 threads = QS channel quads x NTG tap
// groups covering all 16 taps of a 4*QS channel slab; the block walks cpb
// consecutive cells.  dz_l is loaded by each of the NTG tap-group threads
// of a quad (served by L1 after the first).
// ---------------------------------------------------------------------------
template <int DT, int LMAX, int TPT>
__global__ __launch_bounds__(kBlock) void materialise_kernel(const void* __restrict__ base, PtrPack dz, PtrPack beta,
                                                             int wdt, void* __restrict__ out, int L, int64_t ncells,
                                                             int G, int C, int64_t cpb) {
  constexpr int NTG = kK / TPT;
  constexpr int QS = kBlock / NTG;
  const int t = threadIdx.x;
  const int g = t / QS;
  const int c0 = (blockIdx.y * QS + (t - g * QS)) * 4;
  if (c0 >= C) return;
  const int tap0 = g * TPT;
  const int sy = tap0 / kS;
  const int sx0 = tap0 % kS;

  float bw[LMAX][TPT][4];
#pragma unroll
  for (int l = 0; l < LMAX; ++l)
#pragma unroll
    for (int j = 0; j < TPT; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        bw[l][j][v] = (l < L) ? load_w(beta.p[l], wdt, static_cast<int64_t>(c0 + v) * kK + tap0 + j) : 0.f;

  const int64_t cb = static_cast<int64_t>(blockIdx.x) * cpb;
  const int64_t ce = std::min(ncells, cb + cpb);
  for (int64_t cell = cb; cell < ce; ++cell) {
    const int64_t o = tap_offset(cell, G, C, sy, sx0, c0);
    float acc[TPT][4];
    if (base != nullptr) {
#pragma unroll
      for (int j = 0; j < TPT; ++j) load_vec<DT, 4>(base, o + j * C, acc[j]);
    } else {
#pragma unroll
      for (int j = 0; j < TPT; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[j][v] = 0.f;
    }
    const int64_t zo = cell * C + c0;
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      if (l < L) {
        float d[4];
        load_vec<DT, 4>(dz.p[l], zo, d);
#pragma unroll
        for (int j = 0; j < TPT; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[j][v] = fmaf(bw[l][j][v], d[v], acc[j][v]);
      }
    }
#pragma unroll
    for (int j = 0; j < TPT; ++j) store_vec<DT, 4>(out, o + j * C, acc[j]);
  }
}

// ---------------------------------------------------------------------------
// MULTI-WEIGHT READ: out_l[cell,c] = sum_k w_l[c,k] g[cell,k,c]
// Thread = 4 channels x 16 taps x LC layers; the LC x 16 x 4 weights stay in
// VGPRs.  Block = QS quads x NLG layer groups (at most 256 threads); the NLG
// groups of a quad read the same g run (L1 hits after the first).
// ---------------------------------------------------------------------------
template <int DT, int LC>
__global__ __launch_bounds__(kBlock) void read_multi_kernel(const void* __restrict__ g, PtrPack w, int wdt, PtrPack out,
                                                          int L, int QS, int64_t ncells, int G, int C, int64_t cpb) {
  const int t = threadIdx.x;
  const int lg = t / QS;
  const int c0 = (blockIdx.y * QS + (t - lg * QS)) * 4;
  const int l0 = lg * LC;
  if (c0 >= C || l0 >= L) return;
  const int nl = std::min(LC, L - l0);

  float wr[LC][kK][4];
#pragma unroll
  for (int i = 0; i < LC; ++i)
#pragma unroll
    for (int k = 0; k < kK; ++k)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        wr[i][k][v] = (i < nl) ? load_w(w.p[l0 + i], wdt, static_cast<int64_t>(c0 + v) * kK + k) : 0.f;

  const int64_t row = static_cast<int64_t>(G) * kS * C;
  const int64_t cb = static_cast<int64_t>(blockIdx.x) * cpb;
  const int64_t ce = std::min(ncells, cb + cpb);
  for (int64_t cell = cb; cell < ce; ++cell) {
    const int64_t o = tap_offset(cell, G, C, 0, 0, c0);
    float acc[LC][4];
#pragma unroll
    for (int i = 0; i < LC; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][v] = 0.f;
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      float gv[4];
      load_vec<DT, 4>(g, o + (k / kS) * row + (k % kS) * C, gv);
#pragma unroll
      for (int i = 0; i < LC; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][v] = fmaf(gv[v], wr[i][k][v], acc[i][v]);
    }
#pragma unroll
    for (int i = 0; i < LC; ++i)
      if (i < nl) store_vec<DT, 4>(const_cast<void*>(out.p[l0 + i]), cell * C + c0, acc[i]);
  }
}

// ---------------------------------------------------------------------------
// CELL WEIGHT GRADIENT, stage 1: per-block partial sums
//   partial[bx, l, c, k] = sum_{cells of block bx} high[cell,k,c] low_l[cell,c]
// Same thread mapping as materialise_kernel; the LMAX x TPT x 4 accumulators
// stay in VGPRs for the whole cell range of the block.
// ---------------------------------------------------------------------------
template <int DT, int LMAX, int TPT>
__global__ __launch_bounds__(kBlock) void wgrad_partial_kernel(const void* __restrict__ high, PtrPack low,
                                                               float* __restrict__ partial, int L, int64_t ncells,
                                                               int G, int C, int64_t cpb) {
  constexpr int NTG = kK / TPT;
  constexpr int QS = kBlock / NTG;
  const int t = threadIdx.x;
  const int g = t / QS;
  const int c0 = (blockIdx.y * QS + (t - g * QS)) * 4;
  if (c0 >= C) return;
  const int tap0 = g * TPT;
  const int sy = tap0 / kS;
  const int sx0 = tap0 % kS;

  float acc[LMAX][TPT][4];
#pragma unroll
  for (int l = 0; l < LMAX; ++l)
#pragma unroll
    for (int j = 0; j < TPT; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[l][j][v] = 0.f;

  const int64_t cb = static_cast<int64_t>(blockIdx.x) * cpb;
  const int64_t ce = std::min(ncells, cb + cpb);
  for (int64_t cell = cb; cell < ce; ++cell) {
    const int64_t o = tap_offset(cell, G, C, sy, sx0, c0);
    float h[TPT][4];
#pragma unroll
    for (int j = 0; j < TPT; ++j) load_vec<DT, 4>(high, o + j * C, h[j]);
    const int64_t zo = cell * C + c0;
#pragma unroll
    for (int l = 0; l < LMAX; ++l) {
      if (l < L) {
        float d[4];
        load_vec<DT, 4>(low.p[l], zo, d);
#pragma unroll
        for (int j = 0; j < TPT; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[l][j][v] = fmaf(h[j][v], d[v], acc[l][j][v]);
      }
    }
  }
  float* dst = partial + static_cast<int64_t>(blockIdx.x) * L * C * kK;
#pragma unroll
  for (int l = 0; l < LMAX; ++l) {
    if (l < L) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
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

// Zero fill by a kernel rather than hipMemsetAsync, so that callers may
// capture these launches in a HIP graph.
__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

// Stage 2: out[i] = sum_{p < nparts} partial[p, i] in ascending p.
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ partial, int nparts,
                                                              int64_t n, float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int p = 0; p < nparts; ++p) s += partial[static_cast<int64_t>(p) * n + i];
  out[i] = s;
}

// ---------------------------------------------------------------------------
// GAMMA: gamma[l, c] = sum_k alpha[c,k] beta_l[c,k]
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

// ---------------------------------------------------------------------------
// RECURRENCE: z_next = fma(gamma, dz, z).  Block = 64 channel quads x 4 row
// lanes; each thread keeps its 4 gammas and walks rows with stride 4.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void recur_fwd_kernel(const void* __restrict__ z, const void* __restrict__ dz,
                                                        const void* __restrict__ gamma, int gdt,
                                                        void* __restrict__ zn, int64_t rows, int C, int64_t rpb) {
  const int t = threadIdx.x;
  const int c0 = (blockIdx.x * 64 + (t & 63)) * 4;
  if (c0 >= C) return;
  float gm[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) gm[v] = load_w(gamma, gdt, c0 + v);
  const int64_t rb = static_cast<int64_t>(blockIdx.y) * rpb;
  const int64_t re = std::min(rows, rb + rpb);
  for (int64_t r = rb + (t >> 6); r < re; r += 4) {
    const int64_t o = r * C + c0;
    float a[4], d[4];
    load_vec<DT, 4>(z, o, a);
    load_vec<DT, 4>(dz, o, d);
#pragma unroll
    for (int v = 0; v < 4; ++v) a[v] = fmaf(gm[v], d[v], a[v]);
    store_vec<DT, 4>(zn, o, a);
  }
}

// RECURRENCE BACKWARD: gdz = gamma * g; partial[4*by + lane_row, c] = sum g*dz
template <int DT>
__global__ __launch_bounds__(256) void recur_bwd_kernel(const void* __restrict__ g, const void* __restrict__ dz,
                                                        const void* __restrict__ gamma, int gdt,
                                                        void* __restrict__ gdz, float* __restrict__ partial,
                                                        int64_t rows, int C, int64_t rpb) {
  const int t = threadIdx.x;
  const int c0 = (blockIdx.x * 64 + (t & 63)) * 4;
  if (c0 >= C) return;
  float gm[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) gm[v] = load_w(gamma, gdt, c0 + v);
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  const int64_t rb = static_cast<int64_t>(blockIdx.y) * rpb;
  const int64_t re = std::min(rows, rb + rpb);
  for (int64_t r = rb + (t >> 6); r < re; r += 4) {
    const int64_t o = r * C + c0;
    float a[4], d[4], o4[4];
    load_vec<DT, 4>(g, o, a);
    load_vec<DT, 4>(dz, o, d);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      o4[v] = gm[v] * a[v];
      s[v] = fmaf(a[v], d[v], s[v]);
    }
    store_vec<DT, 4>(gdz, o, o4);
  }
  float* dst = partial + (static_cast<int64_t>(blockIdx.y) * 4 + (t >> 6)) * C + c0;
  *reinterpret_cast<float4*>(dst) = make_float4(s[0], s[1], s[2], s[3]);
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

// Cells per block so that a launch has about `blocks_per_cu` blocks per CU.
int64_t cells_per_block(int64_t ncells, int64_t slabs, int blocks_per_cu) {
  const int64_t target = std::max<int64_t>(1, static_cast<int64_t>(num_cus()) * blocks_per_cu / std::max<int64_t>(1, slabs));
  return std::max<int64_t>(1, (ncells + target - 1) / target);
}

// Launch plan of the weight-gradient kernel, shared with its workspace query.
struct WgradPlan {
  int tpt;
  int slabs;
  int64_t cpb;
  int64_t nbx;
};

WgradPlan wgrad_plan(int64_t ncells, int64_t C, int L) {
  WgradPlan p;
  p.tpt = L <= 12 ? 4 : (L <= 24 ? 2 : 1);
  const int qs = kBlock / (kK / p.tpt);
  p.slabs = static_cast<int>((C / 4 + qs - 1) / qs);
  p.cpb = cells_per_block(ncells, p.slabs, 2);
  p.nbx = ncells > 0 ? (ncells + p.cpb - 1) / p.cpb : 0;
  return p;
}

const int64_t kRecurRowsPerBlock = 256;

template <int DT>
void launch_read(const void* x, const void* w, int wdt, void* z, int64_t ncells, int G, int C, bool vec8,
                 hipStream_t st) {
  const int vec = vec8 ? 8 : 4;
  const int ncv = C / vec;
  const int ncv_blk = std::min(ncv, kBlock);
  const int cpi = kBlock / ncv_blk;
  const int gy = (ncv + ncv_blk - 1) / ncv_blk;
  const int64_t cpb = std::max<int64_t>(cpi, cells_per_block(ncells, gy, 8));
  const dim3 grid(static_cast<unsigned>((ncells + cpb - 1) / cpb), gy);
  const dim3 block(ncv_blk * cpi);
  if (vec8) {
    if constexpr (DT != LTHC_F32)
      read_fwd_kernel<DT, 8><<<grid, block, 0, st>>>(x, w, wdt, z, ncells, G, C, ncv_blk, cpi, cpb);
  } else {
    read_fwd_kernel<DT, 4><<<grid, block, 0, st>>>(x, w, wdt, z, ncells, G, C, ncv_blk, cpi, cpb);
  }
}

template <int DT, int LMAX, int TPT>
void launch_materialise_t(const void* base, const PtrPack& dz, const PtrPack& beta, int wdt, void* out, int L,
                          int64_t ncells, int G, int C, hipStream_t st) {
  constexpr int QS = kBlock / (kK / TPT);
  const int slabs = (C / 4 + QS - 1) / QS;
  const int64_t cpb = cells_per_block(ncells, slabs, 8);
  const dim3 grid(static_cast<unsigned>((ncells + cpb - 1) / cpb), slabs);
  materialise_kernel<DT, LMAX, TPT><<<grid, kBlock, 0, st>>>(base, dz, beta, wdt, out, L, ncells, G, C, cpb);
}

template <int DT>
void launch_materialise(const void* base, const PtrPack& dz, const PtrPack& beta, int wdt, void* out, int L,
                        int64_t ncells, int G, int C, hipStream_t st) {
#define LTHC_MAT(LM, TP) launch_materialise_t<DT, LM, TP>(base, dz, beta, wdt, out, L, ncells, G, C, st)
  if (L <= 1) LTHC_MAT(1, 4);
  else if (L <= 2) LTHC_MAT(2, 4);
  else if (L <= 4) LTHC_MAT(4, 4);
  else if (L <= 8) LTHC_MAT(8, 4);
  else if (L <= 12) LTHC_MAT(12, 4);
  else if (L <= 16) LTHC_MAT(16, 2);
  else if (L <= 24) LTHC_MAT(24, 2);
  else if (L <= 32) LTHC_MAT(32, 1);
  else LTHC_MAT(48, 1);
#undef LTHC_MAT
}

template <int DT, int LMAX, int TPT>
void launch_wgrad_t(const void* high, const PtrPack& low, float* partial, int L, int64_t ncells, int G, int C,
                    const WgradPlan& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.nbx), p.slabs);
  wgrad_partial_kernel<DT, LMAX, TPT><<<grid, kBlock, 0, st>>>(high, low, partial, L, ncells, G, C, p.cpb);
}

template <int DT>
void launch_wgrad(const void* high, const PtrPack& low, float* partial, int L, int64_t ncells, int G, int C,
                  const WgradPlan& p, hipStream_t st) {
#define LTHC_WG(LM, TP) launch_wgrad_t<DT, LM, TP>(high, low, partial, L, ncells, G, C, p, st)
  if (L <= 1) LTHC_WG(1, 4);
  else if (L <= 2) LTHC_WG(2, 4);
  else if (L <= 4) LTHC_WG(4, 4);
  else if (L <= 8) LTHC_WG(8, 4);
  else if (L <= 12) LTHC_WG(12, 4);
  else if (L <= 16) LTHC_WG(16, 2);
  else if (L <= 24) LTHC_WG(24, 2);
  else if (L <= 32) LTHC_WG(32, 1);
  else LTHC_WG(48, 1);
#undef LTHC_WG
}

template <int DT, int LC>
void launch_read_multi_t(const void* g, const PtrPack& w, int wdt, const PtrPack& out, int L, int64_t ncells, int G,
                         int C, hipStream_t st) {
  const int nlg = (L + LC - 1) / LC;
  const int qs = std::max(16, (kBlock / nlg) / 16 * 16);  // qs * nlg <= 256 for nlg <= 16
  const int slabs = (C / 4 + qs - 1) / qs;
  const int64_t cpb = cells_per_block(ncells, slabs, 8);
  const dim3 grid(static_cast<unsigned>((ncells + cpb - 1) / cpb), slabs);
  read_multi_kernel<DT, LC><<<grid, qs * nlg, 0, st>>>(g, w, wdt, out, L, qs, ncells, G, C, cpb);
}

template <int DT>
void launch_read_multi(const void* g, const PtrPack& w, int wdt, const PtrPack& out, int L, int64_t ncells, int G,
                       int C, hipStream_t st) {
  // Two layers per thread keep the 128 weights + accumulators within 256
  // VGPRs (3 would spill); 3 per thread only where 16 groups of 2 are not enough.
  if (L == 1) launch_read_multi_t<DT, 1>(g, w, wdt, out, L, ncells, G, C, st);
  else if (L <= 32) launch_read_multi_t<DT, 2>(g, w, wdt, out, L, ncells, G, C, st);
  else launch_read_multi_t<DT, 3>(g, w, wdt, out, L, ncells, G, C, st);
}

template <typename F>
int dispatch_dtype(int dt, F&& f) {
  switch (dt) {
    case LTHC_F32: f(std::integral_constant<int, LTHC_F32>{}); return LTHC_OK;
    case LTHC_BF16: f(std::integral_constant<int, LTHC_BF16>{}); return LTHC_OK;
    case LTHC_F16: f(std::integral_constant<int, LTHC_F16>{}); return LTHC_OK;
    default: return LTHC_ERR_INVALID;
  }
}

int fill_ptrs(const char* fn, PtrPack& pk, const void* const* src, int L, const char* name, int dt, bool act) {
  if (src == nullptr) return fail(LTHC_ERR_INVALID, fn, std::string(name) + " pointer array is NULL");
  for (int l = 0; l < L; ++l) {
    if (src[l] == nullptr) return fail(LTHC_ERR_INVALID, fn, std::string(name) + "[" + std::to_string(l) + "] is NULL");
    if (act && !aligned(src[l], 4 * esize(dt)))
      return fail(LTHC_ERR_INVALID, fn, std::string(name) + "[" + std::to_string(l) + "] is not aligned to 4 elements");
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

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* lthc_last_error(void) { return g_last_error.c_str(); }

int lthc_abi_version(void) { return 1; }

int lthc_read_fwd(const void* x, int x_dtype, const void* alpha, int w_dtype, void* z, int64_t B, int64_t G, int64_t s,
                  int64_t C, void* stream) {
  static const char* fn = "lthc_read_fwd";
  g_last_error.clear();
  if (int rc = check_geom(fn, B, G, s, C)) return rc;
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (B == 0) return LTHC_OK;
  if (int rc = check_act(fn, x, x_dtype, "x")) return rc;
  if (int rc = check_act(fn, z, x_dtype, "z")) return rc;
  if (alpha == nullptr) return fail(LTHC_ERR_INVALID, fn, "alpha is NULL");
  const int64_t ncells = B * G * G;
  const bool vec8 = x_dtype != LTHC_F32 && C % 8 == 0 && aligned(x, 16) && aligned(z, 16);
  dispatch_dtype(x_dtype, [&](auto d) {
    launch_read<decltype(d)::value>(x, alpha, w_dtype, z, ncells, static_cast<int>(G), static_cast<int>(C), vec8,
                                    static_cast<hipStream_t>(stream));
  });
  return check_launch(fn);
}

int lthc_read_multi_fwd(const void* g, int x_dtype, const void* const* w, int w_dtype, void* const* out, int64_t B,
                        int64_t G, int64_t s, int64_t C, int L, void* stream) {
  static const char* fn = "lthc_read_multi_fwd";
  g_last_error.clear();
  if (int rc = check_geom(fn, B, G, s, C)) return rc;
  if (int rc = check_layers(fn, L)) return rc;
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (B == 0) return LTHC_OK;
  if (int rc = check_act(fn, g, x_dtype, "g")) return rc;
  PtrPack wp, op;
  if (int rc = fill_ptrs(fn, wp, w, L, "w", w_dtype, false)) return rc;
  if (int rc = fill_ptrs(fn, op, const_cast<const void* const*>(out), L, "out", x_dtype, true)) return rc;
  const int64_t ncells = B * G * G;
  dispatch_dtype(x_dtype, [&](auto d) {
    launch_read_multi<decltype(d)::value>(g, wp, w_dtype, op, L, ncells, static_cast<int>(G), static_cast<int>(C),
                                          static_cast<hipStream_t>(stream));
  });
  return check_launch(fn);
}

int lthc_materialise_fwd(const void* base, const void* const* dz, int x_dtype, const void* const* beta, int w_dtype,
                         void* out, int64_t B, int64_t G, int64_t s, int64_t C, int L, void* stream) {
  static const char* fn = "lthc_materialise_fwd";
  g_last_error.clear();
  if (int rc = check_geom(fn, B, G, s, C)) return rc;
  if (int rc = check_layers(fn, L)) return rc;
  if (!valid_dtype(x_dtype) || !valid_dtype(w_dtype)) return fail(LTHC_ERR_INVALID, fn, "unknown dtype code");
  if (B == 0) return LTHC_OK;
  if (base != nullptr)
    if (int rc = check_act(fn, base, x_dtype, "base")) return rc;
  if (int rc = check_act(fn, out, x_dtype, "out")) return rc;
  PtrPack dp, bp;
  if (int rc = fill_ptrs(fn, dp, dz, L, "dz", x_dtype, true)) return rc;
  if (int rc = fill_ptrs(fn, bp, beta, L, "beta", w_dtype, false)) return rc;
  const int64_t ncells = B * G * G;
  dispatch_dtype(x_dtype, [&](auto d) {
    launch_materialise<decltype(d)::value>(base, dp, bp, w_dtype, out, L, ncells, static_cast<int>(G),
                                           static_cast<int>(C), static_cast<hipStream_t>(stream));
  });
  return check_launch(fn);
}

size_t lthc_weight_grad_workspace_bytes(int64_t B, int64_t G, int64_t s, int64_t C, int L) {
  if (B <= 0 || G <= 0 || C <= 0 || L < 1 || s != kS) return 0;
  const WgradPlan p = wgrad_plan(B * G * G, C, L);
  return static_cast<size_t>(p.nbx) * static_cast<size_t>(L) * static_cast<size_t>(C) * kK * sizeof(float);
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
  const WgradPlan p = wgrad_plan(ncells, C, L);
  const size_t need = static_cast<size_t>(p.nbx) * n * sizeof(float);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LTHC_ERR_INVALID, fn, "workspace smaller than lthc_weight_grad_workspace_bytes()");
  if (!aligned(workspace, 16)) return fail(LTHC_ERR_INVALID, fn, "workspace is not 16-byte aligned");
  float* partial = static_cast<float*>(workspace);
  dispatch_dtype(x_dtype, [&](auto d) {
    launch_wgrad<decltype(d)::value>(high, lp, partial, L, ncells, static_cast<int>(G), static_cast<int>(C), p, st);
  });
  if (int rc = check_launch(fn)) return rc;
  reduce_partials_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(partial, static_cast<int>(p.nbx), n, gw);
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
  if (int rc = fill_ptrs(fn, bp, beta, L, "beta", w_dtype, false)) return rc;
  const int64_t n = static_cast<int64_t>(L) * C;
  gamma_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      alpha, bp, w_dtype, gamma, out_dtype, static_cast<int>(C), static_cast<int>(K), L);
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
  const dim3 grid(static_cast<unsigned>((C / 4 + 63) / 64), static_cast<unsigned>((rows + kRecurRowsPerBlock - 1) / kRecurRowsPerBlock));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  dispatch_dtype(x_dtype, [&](auto d) {
    recur_fwd_kernel<decltype(d)::value><<<grid, 256, 0, st>>>(z, dz, gamma, g_dtype, z_next, rows, static_cast<int>(C),
                                                               kRecurRowsPerBlock);
  });
  return check_launch(fn);
}

size_t lthc_recur_bwd_workspace_bytes(int64_t rows, int64_t C) {
  if (rows <= 0 || C <= 0) return 0;
  const int64_t by = (rows + kRecurRowsPerBlock - 1) / kRecurRowsPerBlock;
  return static_cast<size_t>(by * 4 * C) * sizeof(float);
}

int lthc_recur_bwd(const void* g, const void* dz, int x_dtype, const void* gamma, int g_dtype, void* gdz, float* ggamma,
                   int64_t rows, int64_t C, void* workspace, size_t workspace_bytes, void* stream) {
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
  const size_t need = lthc_recur_bwd_workspace_bytes(rows, C);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LTHC_ERR_INVALID, fn, "workspace smaller than lthc_recur_bwd_workspace_bytes()");
  if (!aligned(workspace, 16)) return fail(LTHC_ERR_INVALID, fn, "workspace is not 16-byte aligned");
  const int64_t by = (rows + kRecurRowsPerBlock - 1) / kRecurRowsPerBlock;
  const dim3 grid(static_cast<unsigned>((C / 4 + 63) / 64), static_cast<unsigned>(by));
  float* partial = static_cast<float*>(workspace);
  dispatch_dtype(x_dtype, [&](auto d) {
    recur_bwd_kernel<decltype(d)::value><<<grid, 256, 0, st>>>(g, dz, gamma, g_dtype, gdz, partial, rows,
                                                               static_cast<int>(C), kRecurRowsPerBlock);
  });
  if (int rc = check_launch(fn)) return rc;
  reduce_partials_kernel<<<static_cast<unsigned>((C + 255) / 256), 256, 0, st>>>(partial, static_cast<int>(by * 4), C, ggamma);
  return check_launch(fn);
}

}  // extern "C"
