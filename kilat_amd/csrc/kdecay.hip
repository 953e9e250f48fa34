// kdecay.hip — MI355X (gfx950) kernels and C ABI of the global-decay scan.
//
//   s_t = lam_h * s_{t-1} + V_t,   z_t = (1 - lam_h^(t+1)) / ((1 - lam_h) + 1e-6),   y_t = s_t / z_t
//
// Reference semantics: /root/reference/src/kilat/arc/triton_ops.py:232-247 (full
// sequence) and /root/reference/src/kilat/arc/attention.py:344-360 (one decode
// step).  Declarations and argument contracts: include/kdecay.h.
//
// Full-sequence scan (scan_chunked): one workgroup per chunk of L rows of one
// stream: a (b,h) pair and a group of up to 128 bytes of its channels.  Each lane owns R consecutive rows of one
// 16-byte channel slice and keeps them in registers; the chunk is reduced by a
// sequential pass per lane, a shuffle scan across the lanes of a wavefront and
// an LDS fold across wavefronts.  Chunks of one stream are chained in a single
// pass by decoupled look-back: every chunk publishes its aggregate, then its
// inclusive prefix, as 64-bit words (tag << 32 | float bits), one word per
// channel, so a reader needs no fence: the tag and the value arrive together.
// Workgroups are numbered chunk-major (streams rotated per chunk row, to
// spread each stream over the XCDs), so a chunk only waits on workgroups
// with smaller indices.  The inclusive prefix of chunk c is always the same
// left fold
//     F(c) = lam^L * F(c-1) + agg(c)
// whoever evaluates it, so results are bitwise reproducible run to run.

#include <hip/hip_runtime.h>

#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "kdecay.h"

// The reference rounds lam*s and (lam*s)+v separately (two torch ops).  The
// decode step and the sequential scan keep those two roundings (their state is
// bit-identical to the reference's); nothing is contracted implicitly.  The
// chunked scan, which reassociates the recurrence anyway and is checked to a
// tolerance, fuses each lam*s+v into one explicit fmaf: one rounding instead
// of two, and half the vector instructions of its hot loops.
#pragma clang fp contract(off)

namespace kd {

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

// --------------------------------------------------------------------------
// Element conversion
// --------------------------------------------------------------------------
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(double x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ __bf16 from_f32<__bf16>(float x) { return (__bf16)x; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }
template <>
__device__ __forceinline__ double from_f32<double>(float x) { return (double)x; }

// 16 bytes of T -> 16/sizeof(T) floats.
template <typename T>
__device__ __forceinline__ void unpack16(const uint4& u, float* f);

template <>
__device__ __forceinline__ void unpack16<float>(const uint4& u, float* f) {
  f[0] = __uint_as_float(u.x);
  f[1] = __uint_as_float(u.y);
  f[2] = __uint_as_float(u.z);
  f[3] = __uint_as_float(u.w);
}

template <>
__device__ __forceinline__ void unpack16<__bf16>(const uint4& u, float* f) {
  const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void unpack16<_Float16>(const uint4& u, float* f) {
  const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f16x2 h = __builtin_bit_cast(f16x2, w[k]);
    f[2 * k] = (float)h.x;
    f[2 * k + 1] = (float)h.y;
  }
}

// Two doubles, each rounded to float (round to nearest even), as the
// fp32-arithmetic kernels take every input type.
template <>
__device__ __forceinline__ void unpack16<double>(const uint4& u, float* f) {
  f[0] = (float)__hiloint2double((int)u.y, (int)u.x);
  f[1] = (float)__hiloint2double((int)u.w, (int)u.z);
}

__device__ __forceinline__ unsigned pack2(__bf16*, float a, float b) {
  bf16x2 p;
  p.x = (__bf16)a;
  p.y = (__bf16)b;
  return __builtin_bit_cast(unsigned, p);
}
__device__ __forceinline__ unsigned pack2(_Float16*, float a, float b) {
  f16x2 p;
  p.x = (_Float16)a;
  p.y = (_Float16)b;
  return __builtin_bit_cast(unsigned, p);
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-byte store of data written once and not read back by this kernel
// (non-temporal: it does not displace cached data).
__device__ __forceinline__ void store16_stream(void* p, unsigned a, unsigned b, unsigned c, unsigned d) {
  const u32x4 v = {a, b, c, d};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Store N floats (N = 4 or 8; 2 for double) as N elements of T at p (16-byte aligned).
// Eight floats take two 16-byte stores, each of which covers every other 16
// bytes of the row's range across the lanes: through the cache, whose lines
// the second store completes before they are written back (non-temporal,
// bf16 in / fp32 out at B=8 N=4096 H=12 D=64 took 52.2 us; cached, 29.7 us).
// With 8 lanes per row the scan pairs lanes instead (ChunkScan::store_chunk).
template <typename T, int N>
__device__ __forceinline__ void store_vec(T* p, const float* f) {
  if constexpr (sizeof(T) == 4 && N == 8) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const u32x4 v = {__float_as_uint(f[4 * k]), __float_as_uint(f[4 * k + 1]), __float_as_uint(f[4 * k + 2]),
                       __float_as_uint(f[4 * k + 3])};
      *reinterpret_cast<u32x4*>(p + 4 * k) = v;
    }
  } else if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k)
      store16_stream(p + 4 * k, __float_as_uint(f[4 * k]), __float_as_uint(f[4 * k + 1]),
                     __float_as_uint(f[4 * k + 2]), __float_as_uint(f[4 * k + 3]));
  } else if constexpr (sizeof(T) == 8) {
    static_assert(N == 2, "8-byte outputs are stored 2 at a time");
    const double d0 = (double)f[0], d1 = (double)f[1];
    store16_stream(p, (unsigned)__double2loint(d0), (unsigned)__double2hiint(d0), (unsigned)__double2loint(d1),
                   (unsigned)__double2hiint(d1));
  } else {
    static_assert(N == 8, "2-byte outputs are stored 8 at a time");
    store16_stream(p, pack2((T*)nullptr, f[0], f[1]), pack2((T*)nullptr, f[2], f[3]),
                   pack2((T*)nullptr, f[4], f[5]), pack2((T*)nullptr, f[6], f[7]));
  }
}

// --------------------------------------------------------------------------
// Normaliser, as the reference's torch expression evaluates it:
//   z = (1.0 - lam ** (t+1)) / (1.0 - lam + 1e-6)
// torch's pow(tensor, int scalar) returns lam for e == 1, lam*lam for e == 2,
// (lam*lam)*lam for e == 3, and a float power otherwise.  For e >= 4 this
// takes the float rounding of lam^e evaluated in double by binary
// exponentiation (at most 2*64 double products, relative error < 2^-45, so
// the float result is the correctly rounded power except within 2^-45 of a
// rounding tie).  Every other operation is one rounded fp32 op.
// --------------------------------------------------------------------------
__device__ __forceinline__ double ipow_f64(double x, int64_t e) {
  double r = 1.0;
  while (e > 0) {
    if (e & 1) r *= x;
    x *= x;
    e >>= 1;
  }
  return r;
}

__device__ __forceinline__ float pow_like_torch(float x, int64_t e) {
  if (e == 1) return x;
  if (e == 2) return x * x;
  if (e == 3) return (x * x) * x;
  if (e == 0) return 1.0f;
  return (float)ipow_f64((double)x, e);
}

// Wait until at most N vector memory operations of this wavefront are
// outstanding (vmcnt only; the other counters are left alone).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ float z_of(float lam, int64_t t) {
  const float num = 1.0f - pow_like_torch(lam, t + 1);
  const float den = (1.0f - lam) + 1e-6f;
  return num / den;
}

// The same values with lower latency, for the decode step, where z is on the
// critical path of a launch-latency-bound kernel: for e < 2^16 the binary
// exponentiation is unrolled and branch-free (the same products in the same
// order as ipow_f64; squarings past the top bit do not reach r), 12 steps
// instead of 16 for e < 2^12 (C3 decode step 2.22 -> 2.18 us), and the small
// cases are selects instead of branches.  The scan kernels keep the
// loop: they build their z tables while their rows are in flight, and there
// the shorter form measured 3.7% slower (bf16, B=8 N=4096 H=12 D=64).
// x^e by binary exponentiation for 0 <= e < 2^BITS, unrolled and branch-free
// (the products of ipow_f64, in the same order).
template <int BITS>
__device__ __forceinline__ double ipow_f64_bits(double x, unsigned e) {
  double r = 1.0;
#pragma unroll
  for (int k = 0; k < BITS; ++k) {
    const double rx = r * x;
    r = (e >> k) & 1u ? rx : r;
    x *= x;
  }
  return r;
}

// ipow_f64 with the unrolled form for exponents below 2^16.
__device__ __forceinline__ double ipow_f64_fast(double x, int64_t e) {
  if (e >= 0 && e < (1 << 12)) return ipow_f64_bits<12>(x, (unsigned)e);
  if (e >= 0 && e < (1 << 16)) return ipow_f64_bits<16>(x, (unsigned)e);
  return ipow_f64(x, e);
}

__device__ __forceinline__ float pow_like_torch_fast(float x, int64_t e) {
  const double r = ipow_f64_fast((double)x, e);
  const float p2 = x * x;
  const float p3 = p2 * x;
  return e == 1 ? x : e == 2 ? p2 : e == 3 ? p3 : e == 0 ? 1.0f : (float)r;
}

__device__ __forceinline__ float z_of_fast(float lam, int64_t t) {
  const float num = 1.0f - pow_like_torch_fast(lam, t + 1);
  const float den = (1.0f - lam) + 1e-6f;
  return num / den;
}

// --------------------------------------------------------------------------
// Division by a divisor fixed for the launch: a multiply and a shift
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, theorem 4.2 with N = 31: for 2^(l-1) < d <= 2^l
// and m = ceil(2^(31+l) / d) < 2^32, floor(n * m / 2^(31+l)) = floor(n / d)
// for 0 <= n < 2^31).  A compiled division by a runtime value is a chain of
// about 25 dependent instructions (a 64-bit one about 100); the kernels do
// theirs before their first load.
// --------------------------------------------------------------------------
struct FastDiv {
  uint32_t d, m, s;
  __host__ __device__ uint32_t div(uint32_t n) const { return (uint32_t)(((uint64_t)n * m) >> s); }
  __host__ __device__ uint32_t mod(uint32_t n) const { return n - div(n) * d; }
};

// d >= 1.
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while (l < 32 && ((uint64_t)1 << l) < d) ++l;
  const uint32_t s = 31 + l;
  const uint64_t p = (uint64_t)1 << s;  // s <= 63
  return FastDiv{d, (uint32_t)((p + d - 1) / d), s};
}

// --------------------------------------------------------------------------
// Look-back words and the workspace header
// --------------------------------------------------------------------------
typedef unsigned long long u64;

// Header words (first 256 bytes of the workspace).
//   EPOCH  launch generation: look-back words of older launches never match
//   ERROR  sticky fault word (1: a bounded wait gave up).  Every launch reads
//          it with the epoch (one 64-bit load) and, when it is set, writes
//          NaN to all its outputs instead of trusting the workspace: after a
//          give-up, words of the launch that gave up may carry a later
//          launch's tag, so only a cleared workspace computes again.
//   DONE   workgroups of the running launch that have counted toward the
//          epoch's advance (the forward: each stream's last chunk, directly
//          or through a sub-count; the backward: see ChunkBwd::run)
// From byte 256: kCountSlots sub-counts, 32 bytes apart (count_done_2).
enum { HDR_EPOCH = 0, HDR_ERROR = 1, HDR_DONE = 2 };
constexpr unsigned kCountSlots = 64;
constexpr unsigned kCountBase = 64;    // word index of the first sub-count (byte 256)
constexpr unsigned kCountStride = 8;   // words between sub-counts (32 bytes)
constexpr size_t kHeaderBytes = 4 * (kCountBase + kCountSlots * kCountStride);  // 2304

// The epoch and the error word of a workspace header, as one load.
struct EpochErr {
  unsigned epoch, err;
};

__device__ __forceinline__ EpochErr split_header(u64 w) { return EpochErr{(unsigned)w, (unsigned)(w >> 32)}; }

// Tag of a word published in launch `epoch`: kind 0 = aggregate, 1 = inclusive.
// Zeroed memory (tag 0) never matches a live tag.
__device__ __forceinline__ unsigned tag_of(unsigned epoch, unsigned kind) {
  return (((epoch & 0x3fffffffu) + 1u) << 1) | kind;
}

__device__ __forceinline__ void publish(u64* p, unsigned tag, float v) {
  const u64 w = ((u64)tag << 32) | (u64)__float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ u64 peek(const u64* p) {
  return __hip_atomic_load(const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls before a look-back gives up (well over a second): the kernel then
// exits normally and flags the header instead of hanging.
constexpr int kSpinLimit = 1 << 20;

// Look-back window.  When every workgroup of a launch is resident at once, a
// wider window resolves the chunk chains in fewer polls; when the launch runs
// in several rounds, the chunks a workgroup waits on have mostly finished in
// an earlier round, and reading fewer words per poll wins.  Measured (bf16,
// same-box A/B): B=8 N=4096 H=12 D=64 (768 chunks, one round) window 4
// 18.3 us, 2 18.5 us; B=1 N=65536 H=16 D=128 (4096 chunks, four rounds)
// window 4 96.0 us, 3 94.5 us, 2 93.4 us.
constexpr int kW = 4;        // the whole grid resident at once
constexpr int kWRounds = 2;  // several rounds

// Look-back words of the W chunks before chunk c (c >= 1) for channel d:
// w[k] = word of chunk c-1-k.  The reads are unconditional (a load under a
// branch is waited for at the branch join): where c-1-k < 0 the word of chunk
// 0 is read again, and a fold never gets past chunk 0's word, which is always
// inclusive; a lane past the last channel reads the last channel's words.
template <int W, int DG>
__device__ __forceinline__ void read_window(const u64* base, int c, int d, u64 (&w)[W]) {
  const u64* col = base + (d < DG ? d : DG - 1);
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int ck = c - 1 - k > 0 ? c - 1 - k : 0;
    w[k] = peek(col + (int64_t)ck * DG);
  }
}

// F(c-1) for one channel from the words of the W chunks before chunk c, if
// they determine it: the nearest inclusive word, then the aggregates after
// it folded oldest first (F = mL * F + agg).  Every inclusive word is the same
// left fold from the start of the stream, so the result does not depend on
// which inclusive word is the nearest one.  Returns false when a word the fold
// needs is not (yet) published.
template <int W>
__device__ __forceinline__ bool fold_window(const u64 (&w)[W], unsigned tag_agg, unsigned tag_inc, float mL,
                                            float& carry) {
  int m = -1;
  bool open = true;
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const unsigned tag = (unsigned)(w[k] >> 32);
    if (open && tag == tag_inc) m = k;
    if (tag != tag_agg) open = false;
  }
  if (m < 0) return false;
  float f = __uint_as_float((unsigned)w[m]);
#pragma unroll
  for (int k = W - 1; k >= 0; --k)
    if (k < m) f = __builtin_fmaf(mL, f, __uint_as_float((unsigned)w[k]));
  carry = f;
  return true;
}

// Look-back of wavefront 0 for chunk c (c >= 1): carry[q] = F(c-1) of channel
// lane + 64q.  Re-reads the window until every channel's fold succeeds.  A
// look-back that gives up sets the sticky error word and returns a NaN carry
// for the channels it could not resolve: every output that carry reaches
// (the chunk's rows, its inclusive word, and through it later chunks and the
// final state) is NaN, so a caller that checks its outputs for finite values
// sees the fault, not a plausible wrong number.
template <int W, int DG, int DQ>
__device__ void look_back(const u64* base, int c, unsigned tag_agg, unsigned tag_inc, float mL, unsigned* hdr,
                          int spin_limit, float (&carry)[DQ]) {
  const int lane = threadIdx.x & 63;
  bool done[DQ];
#pragma unroll
  for (int q = 0; q < DQ; ++q) done[q] = lane + 64 * q >= DG;
  for (int spin = 0;; ++spin) {
#pragma unroll
    for (int q = 0; q < DQ; ++q) {
      if (!done[q]) {
        u64 w[W];
        read_window<W, DG>(base, c, lane + 64 * q, w);
        done[q] = fold_window<W>(w, tag_agg, tag_inc, mL, carry[q]);
      }
    }
    bool all = true;
#pragma unroll
    for (int q = 0; q < DQ; ++q) all &= done[q];
    if (__ballot(!all) == 0ull) return;
    if (spin >= spin_limit) {
      __hip_atomic_store(hdr + HDR_ERROR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int q = 0; q < DQ; ++q)
        if (!done[q]) carry[q] = __builtin_nanf("");
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Sum of x over the 64 lanes of the wavefront, in a fixed order (the same
// result on every run): DPP butterflies inside each row of 16 lanes, then the
// four row sums.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f32<0x141>(x);  // row_half_mirror
  x += dpp_f32<0x140>(x);  // row_mirror
  const int xi = __builtin_bit_cast(int, x);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 48)));
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, l);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// wave_sum in double, same fixed order.
__device__ __forceinline__ double wave_sum_f64(double x) {
  x += dpp_f64<0xB1>(x);
  x += dpp_f64<0x4E>(x);
  x += dpp_f64<0x141>(x);
  x += dpp_f64<0x140>(x);
  return (readlane_f64(x, 0) + readlane_f64(x, 16)) + (readlane_f64(x, 32) + readlane_f64(x, 48));
}

// Index of the calling wavefront in its workgroup, as a wavefront-uniform
// (scalar) value: loops and branches on it are then scalar, not exec-masked.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Value of `x` held K row groups below (row groups are S lanes apart, GW per
// wavefront; lanes whose group index is below K get an unspecified value).
// Adjacent groups of up to 16 lanes use a DPP row shift (no LDS traffic);
// anything else a lane permute.
template <int K, int GW, int S>
__device__ __forceinline__ float lane_shr(float x) {
  if constexpr (S == 1 && GW <= 16) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x110 | K, 0xf, 0xf, false));
  } else {
    return __shfl_up(x, K * S, 64);
  }
}

// Inclusive scan of the per-lane states over the GW row groups of a
// wavefront: acc(g) = lam^(R*K) * acc(g - K) + acc(g) for K = 1, 2, 4, ...
// pw[K] holds lam^(R*K).
template <int K, int GW, int VW, int S>
__device__ __forceinline__ void group_scan(float (&acc)[VW], int gw, const float* pw) {
  if constexpr (K < GW) {
    const float m = pw[K];
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float o = lane_shr<K, GW, S>(acc[j]);
      if (gw >= K) acc[j] = __builtin_fmaf(m, o, acc[j]);
    }
    group_scan<2 * K, GW, VW, S>(acc, gw, pw);
  }
}

// --------------------------------------------------------------------------
// Chunked single-pass scan
// --------------------------------------------------------------------------
struct ScanArgs {
  const void* V;
  void* out;
  const float* lam;
  const float* init;  // [B*H*D] or null
  float* fin;         // [B*H*D] or null
  int64_t vb, vh, vn; // element strides of V (d stride 1)
  int64_t ob, oh, on; // element strides of out (d stride 1)
  int64_t H, N, t_offset;
  int64_t D;    // head dim (channels of a (b,h) pair)
  int ng;       // channel groups per head: a stream is (b, h, group)
  int nchunk;   // chunks per stream
  int nstream;  // B*H*ng
  u64* flags;   // [nstream][nchunk][DG] look-back words (null if nchunk == 1)
  unsigned* hdr;
  // Optional: the state after every `state_rows` rows, for the backward pass.
  // states[(bh * nsaved + k) * D + d] = s of channel d of head bh at row
  // k * state_rows - 1 (1 <= k < nsaved = ceil(N / state_rows); entry 0 is
  // not written): by head and channel, so the backward may group a head's
  // channels into streams other than the forward's.
  float* states;
  int64_t state_rows;
  int64_t nsaved;
  // With the states: the backward's terms of every row of every head,
  // rowtab[h * N + t] = (1/z, d(1/z)/dlam) at row t (bwd_row_terms), written
  // by the streams of batch 0, first channel group.
  float2* rowtab;
  int spin_limit;  // polls before a look-back gives up (kSpinLimit unless a test lowers it)
  FastDiv f_nstream, f_ng, f_H;  // division by nstream, ng and H
};

// 16-byte load of data read exactly once (non-temporal: no cache residency).
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Buffer resource over `rows` rows of a stream of DG channels, `stride`
// elements apart (stride >= DG), starting at p: the range ends with the last
// row's channels, so a buffer load of any later row returns zeros without
// touching memory.  Offsets are 32-bit: the host keeps a chunk's rows within
// 2^31 bytes.
template <int DG, typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_buffer(const T* p, int64_t rows, int64_t stride) {
  const int64_t bytes = rows > 0 ? ((rows - 1) * stride + DG) * (int64_t)sizeof(T) : 0;
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(p), (short)0, n, 0x00020000);
}

// 16-byte non-temporal buffer load at byte offset `off`.
__device__ __forceinline__ uint4 load16_buffer(__amdgpu_buffer_rsrc_t r, unsigned off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// The launch epoch from the workspace header, kept in a vector register:
// read through a uniform address, the value was moved to a scalar register
// at once, which waited for the load (and every load issued before it).
// One of n workgroups that each finish a launch's use of the epoch: the
// last of them resets the count and advances the epoch for the next launch.
__device__ __forceinline__ void count_done(unsigned* hdr, unsigned n, unsigned epoch) {
  const unsigned d = __hip_atomic_fetch_add(hdr + HDR_DONE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (d == n - 1u) {
    __hip_atomic_store(hdr + HDR_DONE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(hdr + HDR_EPOCH, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// count_done for n workgroups numbered s = 0..n-1 in two levels: workgroup s
// counts on sub-count s % kCountSlots, and the one that completes a sub-count
// counts on DONE (min(n, kCountSlots) of them).  With every count on one word
// the n atomics of a launch queue on that word at the launch's end.  Measured
// (the forward, bf16 D=64, same-box A/B, us, one word / 64 sub-counts 32
// bytes apart): B=128 N=512 H=12 (1536 streams) 106.6 / 42.7, B=64 N=4096
// H=12 (768) 171.3 / 143.5, B=64 N=1024 H=12 44.1 / 39.4, B=40 N=4096 H=16
// (640) 132.5 / 120.6, B=48 N=4096 H=12 (576) 117.2 / 110.8; 16 sub-counts in
// one 64-byte segment did not help (109.6 at 1536 streams), 16 of them 256
// bytes apart nearly did (46.3).  With fewer streams the second atomic is the
// cost: B=16 N=4096 H=12 (192 streams) 38.4 / 38.7, B=8 (96) 17.36 / 17.59;
// between them no gain (B=20, 24, 32 H=12: 48.6 / 48.7, 57.8 / 57.7, 72.2 /
// 72.0; B=16 H=16, 256 streams: 46.6 / 47.1).
__device__ __forceinline__ void count_done_2(unsigned* hdr, unsigned n, unsigned s, unsigned epoch) {
  const unsigned k = s % kCountSlots;
  const unsigned nk = n / kCountSlots + (k < n % kCountSlots ? 1u : 0u);
  unsigned* c = hdr + kCountBase + k * kCountStride;
  const unsigned d = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (d == nk - 1u) {
    __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    count_done(hdr, n < kCountSlots ? n : kCountSlots, epoch);
  }
}

// Streams up to which the forward counts each stream's last chunk on DONE
// directly (count_done_2 above it).
constexpr int kFwdPerStreamCount = 384;

__device__ __forceinline__ EpochErr read_epoch_v(const unsigned* hdr) {
  unsigned zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  return split_header(__hip_atomic_load(reinterpret_cast<u64*>(const_cast<unsigned*>(hdr)) + zero, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT));
}

// Keeps `x` opaque to the optimiser at this point, so values derived from it
// are recomputed after the barrier rather than held in registers across it.
__device__ __forceinline__ void opaque(uint4& x) {
  asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w));
}

// Pins the values of x at this point of the program: computations feeding
// them are done before it and uses come after it (a row-by-row sweep then
// stays row by row instead of running one chain ahead and holding its values).
template <int N>
__device__ __forceinline__ void pin(float (&x)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("" : "+v"(x[j]));
}

// Stream of item j (0 <= j < nstream) of a chunk row rotated by `rot`.
// Items are numbered row by row (every item of chunk row r precedes every
// item of row r+1), so the chunk an item waits on always has a smaller item
// number, whatever the order inside a row.  Inside a row the streams are
// rotated by a different amount per row: workgroups go to the XCDs round-robin
// by index, so without the rotation, whenever nstream is a multiple of 8,
// every chunk of a stream would run on one XCD and each XCD's traffic would
// stay inside its own streams' address ranges.  Spread over the XCDs, the
// same launches ran 10% faster for B=1 N=65536 H=16 D=128 and about 2% faster
// (and steadier from one allocation to the next) for B=8 N=4096 H=12 D=64.
__device__ __forceinline__ int rotated_stream(int j, int rot, int nstream) {
  const int k = j + rot;  // rot < nstream
  return k >= nstream ? k - nstream : k;
}

// Where item `item` of a launch is: chunk (row of chunks), stream, and the
// stream's (b, h, channel group).  Computed once per workgroup.
struct Pos {
  int chunk, stream, bh, grp, b, h;
};

__device__ __forceinline__ Pos pos_of(const ScanArgs& a, int item) {
  Pos p;
  p.chunk = (int)a.f_nstream.div((uint32_t)item);
  const int j = item - p.chunk * a.nstream;
  p.stream = rotated_stream(j, (int)a.f_nstream.mod((uint32_t)p.chunk), a.nstream);
  p.bh = (int)a.f_ng.div((uint32_t)p.stream);
  p.grp = p.stream - p.bh * a.ng;
  p.b = (int)a.f_H.div((uint32_t)p.bh);
  p.h = p.bh - p.b * (int)a.H;
  return p;
}

// One chunk ("item") of the scan: L rows x DG channels of one stream.  A
// stream is one (b,h) pair and one group of DG channels, at most 128 bytes of
// each row: wider heads are split into independent channel groups, which
// keeps the kernel the same for every head dim and gives long sequences more
// streams and shorter look-back chains.
// TI/TO: element types of V / out.  LPR lanes cover one row slice (DG = LPR * VW);
// each lane owns R consecutive rows of one 16-byte channel slice; NW
// wavefronts per workgroup; W = look-back window; FZ: the small-grid
// normaliser; THR: at most two rows' stores in flight per wavefront.
//
// Items are numbered chunk-major (item = chunk * nstream + j, j rotated to
// the stream by the chunk index; see rotated_stream), so the chunk an item
// waits on always has a smaller item number.
// The backward's terms of one row with exponent e = t + 1, from p = lam^(e-1):
//   x = 1/z = ((1 - lam) + 1e-6) / (1 - lam^e)   (lam^e as z_of takes it)
//   y = d(1/z)/dlam = (e lam^(e-1) ((1 - lam) + 1e-6) - (1 - lam^e)) / (1 - lam^e)^2
// lam^e is p times lam (in double); y's numerator, a small difference of
// nearly equal terms when lam is close to 1, stays in double, and both
// quotients are fp32 divisions.  (Two double-precision power loops and a
// double division per row were most of the table's cost; it is built by
// every workgroup for its chunk's rows, on the critical path after the rows
// arrive.)
__device__ __forceinline__ void bwd_row_terms(float lam, int64_t e, double p, float& x, float& y) {
  const double l = lam;
  const double pe = p * l;
  const float pf = e == 1 ? lam : e == 2 ? lam * lam : e == 3 ? (lam * lam) * lam : (float)pe;
  x = ((1.0f - lam) + 1e-6f) / (1.0f - pf);
  const double A = 1.0 - pe;
  y = (float)((double)e * p * ((1.0 - l) + 1e-6) - A) / (float)(A * A);
}

template <typename TI, typename TO, int LPR, int R, int NW, int W, bool FZ, bool THR>
struct ChunkScan {
  static constexpr int VW = 16 / (int)sizeof(TI);  // channels per lane
  static constexpr int DG = LPR * VW;  // channels of one stream
  static constexpr int GW = 64 / LPR;  // row groups per wavefront
  static constexpr int G = NW * GW;    // row groups per chunk
  static constexpr int L = G * R;      // rows per chunk
  static constexpr int NT = NW * 64;
  static constexpr int DQ = (DG + 63) / 64;
  static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "LPR must divide 64");
  static_assert(DG <= 64, "wavefront 0 holds one channel of the stream per lane");
  static_assert(G + 1 <= NT, "power table is filled one entry per thread");

  struct Smem {
    alignas(16) float rz[L];  // 1 / z of each row of the chunk
    float pw[G + 1];  // lam^(R*k), k = 0..G
    float wt[NW][DG];  // per-wavefront totals (zero carry in)
    float carry[DG];   // F(chunk - 1)
  };

  // Issue the loads of this lane's R rows of `item`.  Rows past the end of
  // the sequence read row N-1 instead: the loads stay unconditional (a load
  // under a branch gets a full memory wait at the branch join, serialising
  // the R loads), and rows past the end only ever feed later rows past the
  // end and the last chunk's aggregate, which is never published.
  //
  // Returns the item's decay factor, loaded first: memory operations retire
  // in issue order, so its first use then waits for it alone, not for the
  // rows, and the per-head tables are computed while the rows are in flight.
  // `init` receives the carry-in state of channel `lane` of the stream (the
  // caller's initial state on chunk 0, else 0).  It is loaded here, ahead of
  // the rows and unconditionally (a.lam stands in when there is nothing to
  // load): loaded later, under a condition, it left the compiler unsure at the
  // look-back's join whether the load was still pending, and it waited there
  // for every memory operation, the chunk's own look-back publishes included
  // (a device-scope store round trip on every chunk's critical path).
  __device__ static float load(const ScanArgs& a, const Pos& p, uint4 (&raw)[R], float& init) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int chunk = p.chunk;
    const int64_t bh = p.bh, grp = p.grp, b = p.b, h = p.h;
    const float lam = a.lam[h];
    {
      const bool has = chunk == 0 && a.init != nullptr;
      const float* ip = has ? a.init + bh * a.D + grp * DG + (lane < DG ? lane : DG - 1) : a.lam;
      const float v = *ip;
      init = has ? v : 0.0f;
    }
    const int ds = lane % LPR, gw = lane / LPR;
    const int64_t rbase = (int64_t)chunk * L + (int64_t)(wave * GW + gw) * R;
    const TI* vp = static_cast<const TI*>(a.V) + b * a.vb + h * a.vh + grp * DG + (int64_t)ds * VW;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t r = rbase + i < a.N ? rbase + i : a.N - 1;
      raw[i] = load16_stream(vp + r * a.vn);
    }
    return lam;
  }

  // Scan `item` from its loaded rows and store its outputs.  `eh` holds the
  // launch generation every workgroup read before publishing anything and
  // the workspace's sticky error word.  Tables, chunk reduction and
  // look-back: st = the state before this lane's first row.
  __device__ static void scan_chunk(const ScanArgs& a, const Pos& p, uint4 (&raw)[R], float lam, float init,
                                    EpochErr eh, Smem& sm, float (&st)[VW]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool multi = a.nchunk > 1;
    const int chunk = p.chunk, stream = p.stream;
    const int64_t bh = p.bh, grp = p.grp;
    const int64_t c0 = bh * a.D + grp * DG;  // channel 0 of this stream in [B*H*D] state arrays
    const int64_t row0 = (int64_t)chunk * L;
    const bool last = chunk == a.nchunk - 1;
    const int ds = lane % LPR, gw = lane / LPR;
    const int g = wave * GW + gw;

    // Per-head tables, while the rows are in flight.  (The barrier in front
    // of them measured 1.5% faster at B=8 N=4096 H=12 D=64 bf16 than none.)
    __syncthreads();
    if (tid <= G) sm.pw[tid] = pow_like_torch(lam, (int64_t)tid * R);
    for (int r = tid; r < L; r += NT) {
      if (row0 + r < a.N) sm.rz[r] = 1.0f / (FZ ? z_of_fast(lam, a.t_offset + row0 + r) : z_of(lam, a.t_offset + row0 + r));
    }

    // Sequential pass over the lane's rows (zero carry in).
    float acc[VW];
#pragma unroll
    for (int j = 0; j < VW; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      float v[VW];
      unpack16<TI>(raw[i], v);
#pragma unroll
      for (int j = 0; j < VW; ++j) acc[j] = __builtin_fmaf(lam, acc[j], v[j]);
    }
    __syncthreads();  // tables

    // Inclusive scan over the row groups of the wavefront (adjacent lanes).
    group_scan<1, GW, VW, LPR>(acc, gw, sm.pw);
    if (gw == GW - 1) {
#pragma unroll
      for (int j = 0; j < VW; ++j) sm.wt[wave][ds * VW + j] = acc[j];
    }
    // State before this lane's first row, zero carry into the wavefront.
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float o = lane_shr<1, GW, LPR>(acc[j]);
      acc[j] = gw > 0 ? o : 0.0f;
    }
    __syncthreads();

    // Carry into the chunk: wavefront 0 publishes and looks back.
    const float mW = sm.pw[GW];
    // A workspace whose error word is set may hold words tagged for this
    // launch by the launch that gave up: wavefront 0 then takes the carry as
    // NaN (every output of the chunk, its inclusive word and through it the
    // later chunks become NaN), waits for nothing and does not count toward
    // the epoch's advance (so the epoch every workgroup reads stays the same
    // and no poisoned launch waits for words it will never see).
    bool poisoned = false;
    if (wave == 0) {
      const float mL = sm.pw[G];
      const unsigned tag_agg = tag_of(eh.epoch, 0u), tag_inc = tag_of(eh.epoch, 1u);
      poisoned = __builtin_amdgcn_readfirstlane(eh.err) != 0;
      u64* base = multi ? a.flags + (int64_t)stream * a.nchunk * DG : nullptr;
      float agg[DQ], carry[DQ];
#pragma unroll
      for (int q = 0; q < DQ; ++q) {
        const int d = lane + 64 * q;
        agg[q] = 0.0f;
        carry[q] = 0.0f;
        if (d < DG) {
#pragma unroll
          for (int w = 0; w < NW; ++w) agg[q] = __builtin_fmaf(mW, agg[q], sm.wt[w][d]);
          if (q == 0) carry[q] = init;  // DG <= 64: one channel per lane
          if (chunk > 0 && !last) publish(base + (int64_t)chunk * DG + d, tag_agg, agg[q]);
        }
      }
      if (poisoned) {
#pragma unroll
        for (int q = 0; q < DQ; ++q) carry[q] = __builtin_nanf("");
      } else if (chunk > 0) {
        look_back<W, DG, DQ>(base, chunk, tag_agg, tag_inc, mL, a.hdr, a.spin_limit, carry);
      }
#pragma unroll
      for (int q = 0; q < DQ; ++q) {
        const int d = lane + 64 * q;
        if (d < DG) {
          if (multi && !last) publish(base + (int64_t)chunk * DG + d, tag_inc, __builtin_fmaf(mL, carry[q], agg[q]));
          sm.carry[d] = carry[q];
        }
      }
    }
    // Training forward: the backward's terms of this chunk's rows, once per
    // head, by the other wavefronts while wavefront 0 looks back.
    if constexpr (NW > 1) {
      if (a.rowtab && p.b == 0 && grp == 0 && wave > 0) {
        for (int r = tid - 64; r < L; r += NT - 64) {
          const int64_t row = row0 + r;
          if (row < a.N) {
            const int64_t t = a.t_offset + row;
            float x, y;
            bwd_row_terms(lam, t + 1, ipow_f64((double)lam, t), x, y);
            a.rowtab[p.h * a.N + row] = make_float2(x, y);
          }
        }
      }
    }
    __syncthreads();

    // The last chunk of a stream has seen, through its look-back, a word of
    // every earlier chunk of the stream, each written after its workgroup
    // read the epoch.  When the last chunk of every stream is here, every
    // workgroup of this launch has read the epoch (each holds at least one
    // item): advance it for the next launch.  (Counted after the stores
    // instead, C2 measured 1.7% slower and the small grids 2.5%.)
    if (multi && last && tid == 0 && !poisoned) {
      if (a.nstream <= kFwdPerStreamCount)
        count_done(a.hdr, (unsigned)a.nstream, eh.epoch);
      else
        count_done_2(a.hdr, (unsigned)a.nstream, (unsigned)stream, eh.epoch);
    }

    // The lane's true start state.
    float ew[VW];  // state before this wavefront's first row, zero carry into the chunk
#pragma unroll
    for (int j = 0; j < VW; ++j) ew[j] = 0.0f;
    for (int w = 0; w < wave; ++w) {
#pragma unroll
      for (int j = 0; j < VW; ++j) ew[j] = __builtin_fmaf(mW, ew[j], sm.wt[w][ds * VW + j]);
    }
    const float mg = sm.pw[g];
    const float mgw = sm.pw[gw];
#pragma unroll
    for (int j = 0; j < VW; ++j) st[j] = __builtin_fmaf(mg, sm.carry[ds * VW + j], __builtin_fmaf(mgw, ew[j], acc[j]));
  }

  // Re-run the lane's rows from st and store y (and the optional outputs).
  __device__ static void store_chunk(const ScanArgs& a, const Pos& p, uint4 (&raw)[R], float lam, float (&st)[VW],
                                     const Smem& sm) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = p.chunk, stream = p.stream;
    const int bh = p.bh, grp = p.grp, b = p.b, h = p.h;
    const int64_t c0 = (int64_t)bh * a.D + grp * DG;
    const int ds = lane % LPR, gw = lane / LPR;
    const int g = wave * GW + gw;
    const int64_t rbase = (int64_t)chunk * L + (int64_t)g * R;
    TO* op = static_cast<TO*>(a.out) + b * a.ob + h * a.oh + grp * DG + (int64_t)ds * VW + rbase * a.on;
    // fp32 output of a 2-byte V, 8 lanes per row: a lane's 8 outputs are 32
    // bytes, and a row's 256 bytes two 128-byte lines.  Stored as they lie,
    // each of the two store instructions would cover every other 16 bytes of
    // both lines.  Paired, lanes 0-3 and 4-7 swap halves so that the first
    // instruction writes the first line whole (lane ds < 4 its own first
    // half at 8 ds, lane ds >= 4 its partner's second half at 8 (7 - ds) + 4)
    // and the second the second line.  B=8 N=4096 H=12 D=64 bf16 in: 30.8 ->
    // 28.6 us; B=8 N=1024 H=6 D=128 12.5 -> 9.7 us; B=2 N=1000 H=3 D=128
    // (48 workgroups) 7.4 -> 7.8 us (same-box A/B against the cached unpaired
    // stores, identical outputs).
    constexpr bool kPairedStores = sizeof(TO) == 4 && VW == 8 && LPR == 8;
    TO* const op1 = op - ds * VW + (ds < 4 ? 8 * ds : 60 - 8 * ds);
    TO* const op2 = op - ds * VW + (ds < 4 ? 56 - 8 * ds : 8 * ds + 4);
    // Rows of this lane inside the sequence, and which of them (if any) is
    // row N-1, as 32-bit values (no 64-bit compare per row).
    const int nvalid = a.N - rbase >= R ? R : (a.N - rbase > 0 ? (int)(a.N - rbase) : 0);
    const int64_t fr = a.N - 1 - rbase;
    const int ifin = a.fin != nullptr && fr >= 0 && fr < R ? (int)fr : -1;
    // Row i: advance the state, scale by 1/z, store.  Throttled (THR), the
    // stores of a chunk's first rows would otherwise queue in the CU's memory
    // path ahead of the look-back polls and row loads of the other
    // workgroups on the CU, which then wait behind them.
    // The lane's normalisers, read at once (one LDS read per row left each
    // row waiting on its own read: 0.5-1.4% on every shape measured).
    static_assert(R % 4 == 0, "normalisers are read four at a time");
    float rzl[R];
#pragma unroll
    for (int k = 0; k < R / 4; ++k) {
      const float4 q = *reinterpret_cast<const float4*>(&sm.rz[g * R + 4 * k]);
      rzl[4 * k] = q.x;
      rzl[4 * k + 1] = q.y;
      rzl[4 * k + 2] = q.z;
      rzl[4 * k + 3] = q.w;
    }
    auto row = [&](int i) {
      float v[VW], y[VW];
      opaque(raw[i]);
      unpack16<TI>(raw[i], v);
      const float rz = rzl[i];
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        st[j] = __builtin_fmaf(lam, st[j], v[j]);
        y[j] = st[j] * rz;
      }
      if constexpr (kPairedStores) {
        // Lane ds and lane 7 - ds (DPP half-row mirror) trade the half of
        // their 32 bytes that lies in the other's 128-byte line.
        const bool lo = ds < 4;
        float s1[4], s2[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float snd = lo ? y[4 + k] : y[k];
          const float r = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(snd), 0x141, 0xf, 0xf, false));
          s1[k] = lo ? y[k] : r;
          s2[k] = lo ? r : y[4 + k];
        }
        store16_stream(op1 + (int64_t)i * a.on, __float_as_uint(s1[0]), __float_as_uint(s1[1]), __float_as_uint(s1[2]),
                       __float_as_uint(s1[3]));
        store16_stream(op2 + (int64_t)i * a.on, __float_as_uint(s2[0]), __float_as_uint(s2[1]), __float_as_uint(s2[2]),
                       __float_as_uint(s2[3]));
      } else {
        store_vec<TO, VW>(op + (int64_t)i * a.on, y);
      }
      if constexpr (THR) {
        if (i >= 2) wait_vmcnt<2 * (VW * (int)sizeof(TO) / 16)>();
      }
    };
    if (nvalid == R && (ifin < 0 || ifin == R - 1)) {
      // Every row of the lane inside the sequence and row N-1, if the lane
      // holds it, its last: no per-row guard (each guard made the compiler
      // merge the state with copies at its join: B=8 N=4096 H=12 D=64 1.5%
      // and B=8 N=1024 H=6 4% slower with the guarded loop alone).  The
      // final state is then the state after the loop.  (Sent down the
      // guarded loop, the lanes holding row N-1 made their wavefront run
      // both loops, in the last chunk of every stream: C2 with the final
      // state 18.7 against 17.5 us without.)
#pragma unroll
      for (int i = 0; i < R; ++i) row(i);
      if (ifin == R - 1) {
#pragma unroll
        for (int j = 0; j < VW; ++j) a.fin[c0 + ds * VW + j] = st[j];
      }
    } else {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        if (i < nvalid) {
          row(i);
          if (i == ifin) {
#pragma unroll
            for (int j = 0; j < VW; ++j) a.fin[c0 + ds * VW + j] = st[j];
          }
        }
      }
    }
    if (a.states) {
      const int64_t e = rbase + R;  // st is the state at row e - 1
      if (e < a.N && e % a.state_rows == 0) {
        float* sp = a.states + ((int64_t)bh * a.nsaved + e / a.state_rows) * a.D + grp * DG + ds * VW;
#pragma unroll
        for (int j = 0; j < VW; ++j) sp[j] = st[j];
      }
    }
  }

  __device__ static void process(const ScanArgs& a, const Pos& p, uint4 (&raw)[R], float lam, float init,
                                 EpochErr eh, Smem& sm) {
    float st[VW];
    scan_chunk(a, p, raw, lam, init, eh, sm, st);
    store_chunk(a, p, raw, lam, st, sm);
  }
};

// The launch epoch and the error word, read by every thread before it loads
// any rows (so that waiting for them does not wait for the rows).  A launch
// of one chunk per stream has no workspace.
__device__ __forceinline__ EpochErr read_epoch(const ScanArgs& a) {
  if (a.nchunk <= 1) return EpochErr{0u, 0u};
  return split_header(__hip_atomic_load(reinterpret_cast<u64*>(a.hdr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// One item per workgroup: workgroup b owns item b.  An item only waits on
// items with smaller indices, which are dispatched first (workgroups are
// dispatched in index order on each XCD), so the smallest unfinished item
// can always run: no co-residency requirement and no ticket counter.
template <typename TI, typename TO, int LPR, int R, int NW, int W, int WPE, bool FZ, bool THR>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, 8)))
void scan_chunked(ScanArgs a) {
  using CS = ChunkScan<TI, TO, LPR, R, NW, W, FZ, THR>;
  __shared__ typename CS::Smem sm;
  const EpochErr eh = read_epoch(a);
  const Pos p = pos_of(a, (int)blockIdx.x);
  uint4 raw[R];
  float init;
  const float lam = CS::load(a, p, raw, init);
  CS::process(a, p, raw, lam, init, eh, sm);
}

// --------------------------------------------------------------------------
// Backward of the full-sequence scan
// --------------------------------------------------------------------------
// For y_t = s_t / z_t, s_t = lam * s_{t-1} + v_t and upstream gradient gy:
//   u_t  = gy_t / z_t  (+ the final-state gradient at t = N-1)
//   g_t  = u_t + lam * g_{t+1}           (reverse-time decay scan; g_N = 0)
//   dV_t = g_t,  d(init) = lam * g_0
//   dlam = sum_t g_t * s_{t-1} + sum_t gy_t * s_t * d(1/z_t)/dlam
// One workgroup per chunk, chunks taken from the end of the sequence: dV uses
// the forward scan's look-back with the chunk order reversed.  s is
// recomputed inside each chunk from the state the forward pass saved at the
// chunk's first row (ScanArgs::states), so no second look-back is needed.
//
// dlam needs no row of V after the look-back.  For a lane's R rows t0 + i,
// with sl / gl the lane-local scans started from zero (forward from the
// lane's first row, reverse from its last), s_in = s_{t0-1} and
// g_out = g_{t0+R}:
//   sum_i g s_{t-1} = P + s_in Q1 + g_out Q2 + s_in g_out R lam^R
//   P  = sum_i u_i wl_i,  wl_i = lam wl_{i-1} + sl_{i-1}   (wl_{-1} = sl_{-1} = 0)
//   Q1 = sum_i u_i (i+1) lam^i,  Q2 = lam wl_{R-1}
//   sum_i gy z' s = sum_i e_i sl_i + s_in sum_i e_i lam^(i+1),  e_i = gy_i d(1/z)/dlam
// P and the sl/wl terms take one forward sweep over V and gy together; V's
// registers are free after it.  The g_out terms split into the chunk-local
// part (known before the look-back) and carry * K, with K summed over the
// chunk's lanes per channel, so after the look-back one product per channel
// finishes the chunk's dlam partial.  Only gy is held across the look-back,
// for the dV pass.  Each chunk writes its dlam partial; the last workgroup of
// each head sums them in a fixed order (deterministic).
struct BwdArgs {
  const void* V;
  const void* gy;
  void* dv;
  const float* lam;
  const float* init;    // [B*H*D] or null
  const float* states;  // forward states at chunk starts (ScanArgs::states layout, by head and channel), null if nchunk == 1
  const float2* rowtab; // the training forward's per-row terms (ScanArgs::rowtab), null if nchunk == 1
  const float* gfin;    // [B*H*D] or null: gradient of the final state
  float* dinit;         // [B*H*D] or null
  float* dlam;          // [H]
  u64* partial;         // [nchunk * nstream] dlam partial per chunk (rc * nstream + stream), epoch-tagged words
  int64_t vb, vh, vn, gb, gh, gn, db, dh, dn;
  int64_t B, H, N, t_offset, D;
  int ng, nchunk, nstream;
  int64_t nsaved;
  u64* flags;
  unsigned* hdr;
  int spin_limit;  // as ScanArgs::spin_limit, for the look-back and the dlam reduction
  int ndone;       // workgroups that count toward the epoch's advance (ChunkBwd::run)
  int per_stream;  // 1: the first chunk of every stream counts instead
  FastDiv f_nstream, f_ng, f_H, f_nchunk;  // division by nstream, ng, H and nchunk
  // Batch slices (kdecay_scan_bwd): this launch is slice `slice` of `nslice`;
  // the earlier slices' per-head dlam sums, in double ([nslice - 1][H]).
  int slice, nslice;
  double* dlam_slices;
};

// XCDs of the device: workgroups are handed to them round-robin by index, and
// each XCD dispatches its share in index order.
constexpr int kXcds = 8;

// Value of `x` held K row groups above (row groups S lanes apart; lanes with
// gw + K >= GW get an unspecified value).
template <int K, int GW, int S>
__device__ __forceinline__ float lane_shl(float x) {
  if constexpr (S == 1 && GW <= 16) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x100 | K, 0xf, 0xf, false));
  } else {
    return __shfl_down(x, K * S, 64);
  }
}

// Reverse inclusive scan over the GW row groups: acc(g) = acc(g) + lam^(R*K) * acc(g + K).
template <int K, int GW, int VW, int S>
__device__ __forceinline__ void group_scan_rev(float (&acc)[VW], int gw, const float* pw) {
  if constexpr (K < GW) {
    const float m = pw[K];
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float o = lane_shl<K, GW, S>(acc[j]);
      if (gw + K < GW) acc[j] = __builtin_fmaf(m, o, acc[j]);
    }
    group_scan_rev<2 * K, GW, VW, S>(acc, gw, pw);
  }
}

// SL: a launch over a batch slice (kdecay_scan_bwd), whose head sums go
// through BwdArgs::dlam_slices.
template <typename T, int LPR, int R, int NW, int W, bool SL = false>
struct ChunkBwd {
  static constexpr int VW = 16 / (int)sizeof(T);
  static constexpr int DG = LPR * VW;
  static constexpr int GW = 64 / LPR;
  static constexpr int G = NW * GW;
  static constexpr int L = G * R;
  static constexpr int NT = NW * 64;
  static constexpr int DQ = (DG + 63) / 64;
  static constexpr int NR = (L + NT - 1) / NT;  // rows of the table per thread
  // Load the training forward's row terms (BwdArgs::rowtab) instead of
  // computing them, for 1 or 2 rows per thread: the table's power and
  // division chain then no longer delays the first sweep row (2 rows, 16 per
  // lane: C2 27.51 -> 27.11-27.28 us, B=24 N=1024 H=16 28.0 -> 27.5, C4
  // unchanged; 1 row, 128-row chunks: B=8 N=1024 H=6 10.76 -> 10.40, B=2
  // N=4096 H=12 13.81 -> 13.63, B=8 N=2048 H=12 21.14 -> 21.22; gradients
  // bit-identical; same-box A/B on shared buffers).  With 4 rows per thread
  // (D=32 bf16) the eight loads cost more than the chain, and with 8 their
  // registers spilled.
  static constexpr bool kLoadTerms = NR <= 2;
  static_assert(G + 1 <= NT, "power table is filled one entry per thread");

  // Per row of the chunk (i = the row's index in its lane, 0 <= i < R):
  // x = 1/z, y = d(1/z)/dlam, z = x (i+1) lam^i + y lam^(i+1), w = x lam^i
  // (zero for rows past the end).  Entry of row r: rt4[r + r / R], one entry
  // of padding after each lane's R rows: the GW row groups of a wavefront
  // read their own rows' entries at once, R entries (R * 16 bytes) apart,
  // which without the padding all fell into the same LDS banks (an 8-way
  // conflict on every table read of the sweeps).  kq likewise has a padded
  // row: its 64 lanes' writes hit 16-way conflicts with rows of DG floats.
  static constexpr int TS = R + 1;  // table entries per row group
  struct Smem {
    float4 rt4[G * TS];
    float pw[G + 1];   // lam^(R*k)
    float pl[R + 1];   // lam^i
    float wt[NW][DG];  // forward per-wavefront totals
    float rt[NW][DG];  // reverse per-wavefront totals
    float kq[G][DG + 1];  // the carry coefficient K of every lane
    float carry_s[DG]; // state before the chunk's first row
    float carry_g[DG]; // g after the chunk's last row
    float gfin[DG];    // final-state gradient (last chunk only; zero elsewhere)
    double red[NW];    // carry-free dlam partial per wavefront
  };

  // Forward sweep over V and gy together (zero state in): sl = lane-local
  // state, wl = lane-local d(state)/dlam; dq = the sum over the lane's rows
  // and channels of u wl + e sl, with u = gy / z and e = gy d(1/z)/dlam, taken
  // per row as rz * sum_j gy wl + rzp * sum_j gy sl.  From row F0 on it also
  // takes sweep_gy's sums (qz, ra), saving that pass's unpacking of those
  // rows: with few rows per lane from the first row (F0 = 0), with 16 rows
  // from row 8, once the V rows consumed so far have freed the 16 registers
  // the sums take (from row 6 on, 4 bytes spilled and the C2 backward was
  // 3% slower; from row 8, 1% faster than a separate pass over all 16 rows,
  // 27.55 against 27.9 us, same-box A/B).  One row at a time (pin): left
  // free, the compiler ran the whole state chain first and held every row's
  // states.  Each row's table entry is read one row ahead.  fin_i: the
  // lane's row N-1 (final-state gradient), or -1.
  template <int F0>
  __device__ static void sweep_fwd(const uint4 (&rv)[R], uint4 (&rg)[R], float lam, int g, int fin_i, int ds,
                                   const Smem& sm, float (&sl)[VW], float (&wl)[VW], float& dq, float (&qz)[VW],
                                   float (&ra)[VW]) {
    static_assert(F0 < R, "the sweep takes the gy-only sums of its last rows at least");
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      sl[j] = 0.0f;
      wl[j] = 0.0f;
      qz[j] = 0.0f;
      ra[j] = 0.0f;
    }
    dq = 0.0f;
    float4 t = sm.rt4[g * TS];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const float4 tn = sm.rt4[g * TS + (i + 1 < R ? i + 1 : i)];
      float v[VW], gv[VW];
      unpack16<T>(rv[i], v);
      unpack16<T>(rg[i], gv);
      float pw = 0.0f, ps = 0.0f;
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        wl[j] = __builtin_fmaf(lam, wl[j], sl[j]);
        sl[j] = __builtin_fmaf(lam, sl[j], v[j]);
        pw = __builtin_fmaf(gv[j], wl[j], pw);
        ps = __builtin_fmaf(gv[j], sl[j], ps);
        if (i >= F0) {
          qz[j] = __builtin_fmaf(gv[j], t.z, qz[j]);
          ra[j] = __builtin_fmaf(gv[j], t.w, ra[j]);
        }
      }
      dq = __builtin_fmaf(t.x, pw, __builtin_fmaf(t.y, ps, dq));
      if (i == fin_i) {
#pragma unroll
        for (int j = 0; j < VW; ++j) dq = __builtin_fmaf(sm.gfin[ds * VW + j], wl[j], dq);
      }
      t = tn;
      pin(sl);
      pin(wl);
      asm volatile("" : "+v"(dq));
      if (i >= F0) {
        pin(qz);
        pin(ra);
      }
    }
    if (F0 == 0) add_fin(fin_i, ds, sm, qz, ra);
  }

  // The final-state gradient's share of qz and ra (row fin_i of the lane).
  __device__ static void add_fin(int fin_i, int ds, const Smem& sm, float (&qz)[VW], float (&ra)[VW]) {
    if (fin_i >= 0) {
      const float p = sm.pl[fin_i];
      const float c = p * (float)(fin_i + 1);
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float gf = sm.gfin[ds * VW + j];
        qz[j] = __builtin_fmaf(gf, c, qz[j]);
        ra[j] = __builtin_fmaf(gf, p, ra[j]);
      }
    }
  }

  // gy-only sweep over the lane's rows below F1, summed onto the forward
  // sweep's sums of the later rows: qz = Q1 + sum_i e_i lam^(i+1), ra = gl at
  // the lane's first row (zero carry from the right) = sum_i lam^i u_i.
  template <int F1>
  __device__ static void sweep_gy(uint4 (&rg)[R], int g, int fin_i, int ds, const Smem& sm, float (&qz)[VW],
                                  float (&ra)[VW]) {
    float2 tc = *reinterpret_cast<const float2*>(&sm.rt4[g * TS].z);
#pragma unroll
    for (int i = 0; i < F1; ++i) {
      const float2 tn = *reinterpret_cast<const float2*>(&sm.rt4[g * TS + (i + 1 < F1 ? i + 1 : i)].z);
      float gv[VW];
      opaque(rg[i]);
      unpack16<T>(rg[i], gv);
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        qz[j] = __builtin_fmaf(gv[j], tc.x, qz[j]);
        ra[j] = __builtin_fmaf(gv[j], tc.y, ra[j]);
      }
      tc = tn;
      pin(qz);
      pin(ra);
    }
    add_fin(fin_i, ds, sm, qz, ra);
  }

  // Reverse pass with the lane's true g_out: g of every row, stored as dV
  // (rows up to li, the lane's last row inside the sequence).
  __device__ static void sweep_dv(const BwdArgs& a, uint4 (&rg)[R], float lam, int g, int li, int fin_i, int ds,
                                  const Smem& sm, T* dp, float (&gn)[VW]) {
    // Every row of the lane inside the sequence and row N-1, if the lane
    // holds it, its last (the first this pass takes): no per-row guard (C2
    // 29.5 -> 29.3 us, B=1 N=65536 H=16 D=128 146.6 -> 145.2 us), one guarded
    // add of the final-state gradient on the first row.  Only for channel
    // groups of 128 bytes or more: for narrower ones the second loop made one
    // of the kernels spill (D=32 bf16, several rounds, 7% slower).  With 16
    // rows, at most two rows' stores in flight per wavefront, as in the
    // forward (re-measured on shared buffers, us, none / 1 / 2 / 4 rows in
    // flight: C2 28.51 / 27.03 / 27.06 / 27.93, B=24 N=1024 H=16 28.80 /
    // 27.19 / 27.37 / 28.04, C4 145.5 / 146.4 / 145.8 / 145.7), but only
    // when the grid is resident at once: in several rounds a workgroup's slot
    // goes to the next round's only once its stores are done, and those
    // wait behind the next round's reads (stamps at B=16 N=4096 H=12 D=64,
    // two rounds: 7 us from the first-round dV pass to the workgroup's end,
    // against 1.5-3 us in one round).  Unthrottled there (same-box A/B on
    // shared buffers, us, bf16, N=4096 H=12 unless given): D=64 B=16 59.68
    // -> 57.72, B=24 87.95 -> 86.99, B=32 110.05 -> 108.42; D=128 B=8 59.29
    // -> 58.46; C4 145.89 -> 145.50; identical outputs.
    if constexpr (LPR >= 8) {
      if (li == R - 1 && (fin_i < 0 || fin_i == R - 1)) {
#pragma unroll
        for (int i = R - 1; i >= 0; --i) {
          float gv[VW];
          opaque(rg[i]);
          unpack16<T>(rg[i], gv);
          const float rz = sm.rt4[g * TS + i].x;
#pragma unroll
          for (int j = 0; j < VW; ++j) gn[j] = __builtin_fmaf(lam, gn[j], gv[j] * rz);
          if (i == R - 1 && fin_i == R - 1) {
#pragma unroll
            for (int j = 0; j < VW; ++j) gn[j] += sm.gfin[ds * VW + j];
          }
          store_vec<T, VW>(dp + (int64_t)i * a.dn, gn);
          if constexpr (R >= 16 && W != kWRounds) {
            if (i <= R - 3) wait_vmcnt<2>();
          }
          pin(gn);
        }
        return;
      }
    }
#pragma unroll
    for (int i = R - 1; i >= 0; --i) {
      float gv[VW];
      opaque(rg[i]);
      unpack16<T>(rg[i], gv);
      const float rz = sm.rt4[g * TS + i].x;
#pragma unroll
      for (int j = 0; j < VW; ++j) gn[j] = __builtin_fmaf(lam, gn[j], gv[j] * rz);
      if (i == fin_i) {
#pragma unroll
        for (int j = 0; j < VW; ++j) gn[j] += sm.gfin[ds * VW + j];
      }
      if (i <= li) store_vec<T, VW>(dp + (int64_t)i * a.dn, gn);
      pin(gn);
    }
  }

  __device__ static void run(const BwdArgs& a, Smem& sm) {
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const bool multi = a.nchunk > 1;
    const int item = blockIdx.x;
    // rc: position from the end.  The rotation leaves the last row (rc =
    // nchunk-1) unrotated, which reduce_head's choice of workgroup relies on.
    const int rc = (int)a.f_nstream.div((uint32_t)item);
    const int chunk = a.nchunk - 1 - rc;
    const int stream = rotated_stream(item - rc * a.nstream, (int)a.f_nstream.mod((uint32_t)chunk), a.nstream);
    const int bh = (int)a.f_ng.div((uint32_t)stream), grp = stream - bh * a.ng;
    const int b = (int)a.f_H.div((uint32_t)bh), h = bh - b * (int)a.H;
    const int64_t c0 = (int64_t)bh * a.D + grp * DG;
    const int64_t row0 = (int64_t)chunk * L;
    const int ds = lane % LPR, gw = lane / LPR;
    const int g = wave * GW + gw;
    const int gr = g * R;  // the lane's first row within the chunk (rows row0 + gr ...)
    const float lam = a.lam[h];

    // For channel tid < DG: the forward state before the chunk's first row
    // (saved by the forward pass, the initial state, or zero) and the
    // final-state gradient (last chunk only, else zero).  Both loads are
    // issued before the rows and unconditionally (a load under a branch is
    // waited for at the branch join): a.lam stands in where there is nothing
    // to load.
    float cs, cf;
    {
      const int dc = tid < DG ? tid : DG - 1;
      const float* cp = chunk > 0 ? a.states + ((int64_t)bh * a.nsaved + chunk) * a.D + grp * DG + dc
                                  : (a.init ? a.init + c0 + dc : a.lam);
      const bool fin = rc == 0 && a.gfin != nullptr;
      const float* fp = fin ? a.gfin + c0 + dc : a.lam;
      cs = *cp;
      cf = *fp;
      if (chunk == 0 && !a.init) cs = 0.0f;
      if (!fin) cf = 0.0f;
    }
    // The row terms the training forward saved for this thread's rows of the
    // table (below), loaded before the rows so that they arrive first; rows
    // past the end read row N-1, and without saved terms a.lam stands in.
    float tx[NR], ty[NR];
#pragma unroll
    for (int k = 0; k < (kLoadTerms ? NR : 0); ++k) {
      const int rr = tid + k * NT < L ? tid + k * NT : L - 1;  // rows of this chunk only
      const int64_t r = row0 + rr < a.N ? row0 + rr : a.N - 1;
      const float* tp = a.rowtab ? reinterpret_cast<const float*>(a.rowtab + h * a.N + r) : a.lam;
      tx[k] = tp[0];
      ty[k] = (a.rowtab ? tp + 1 : a.lam)[0];
    }

    // Rows of V and gy, through buffer loads whose range ends with the
    // stream's row N-1: rows past the end read as zero (the hardware's range
    // check), so no row index is clamped.  li: index of the lane's last row
    // inside the sequence (R - 1 outside the last chunk).
    const int64_t left = a.N - 1 - row0;  // the chunk's last row inside the sequence
    const int li = left - gr < R - 1 ? (int)(left - gr) : R - 1;
    uint4 rv[R], rg[R];
    {
      const __amdgpu_buffer_rsrc_t bv =
          row_buffer<DG>(static_cast<const T*>(a.V) + b * a.vb + h * a.vh + grp * DG + row0 * a.vn, a.N - row0, a.vn);
      const __amdgpu_buffer_rsrc_t bg =
          row_buffer<DG>(static_cast<const T*>(a.gy) + b * a.gb + h * a.gh + grp * DG + row0 * a.gn, a.N - row0, a.gn);
      const unsigned ov = (unsigned)(((int64_t)g * R * a.vn + ds * VW) * (int64_t)sizeof(T));
      const unsigned og = (unsigned)(((int64_t)g * R * a.gn + ds * VW) * (int64_t)sizeof(T));
      const unsigned sv = (unsigned)(a.vn * (int64_t)sizeof(T)), sg = (unsigned)(a.gn * (int64_t)sizeof(T));
      // Row by row, V then gy: the forward sweep takes them in that order,
      // as they arrive.
#pragma unroll
      for (int i = 0; i < R; ++i) {
        rv[i] = load16_buffer(bv, ov + i * sv);
        rg[i] = load16_buffer(bg, og + i * sg);
      }
    }

    __syncthreads();
    if (tid <= G) sm.pw[tid] = pow_like_torch(lam, (int64_t)tid * R);
    if (tid >= NT - (R + 1)) sm.pl[tid - (NT - (R + 1))] = pow_like_torch(lam, (int64_t)(tid - (NT - (R + 1))));
    {
      // One double-precision power per thread: lam^(e-1) of its first row,
      // times lam^NT for each later row (NT apart).  A thread's rows share
      // their index in the lane (NT is a multiple of R), hence lam^i.
      static_assert(NT % R == 0 && (NT & (NT - 1)) == 0, "rows of a thread");
      const int i = tid % R;
      const float p = pow_like_torch(lam, i);
      const float p1 = p * lam;
      if (kLoadTerms && a.rowtab) {
#pragma unroll
        for (int k = 0; k < NR; ++k) {
          const int r = tid + k * NT;
          if (r < L) {
            const bool in = row0 + r < a.N;
            const float x = in ? tx[k] : 0.0f, y = in ? ty[k] : 0.0f;
            const float w = x * p;
            sm.rt4[r + r / R] = make_float4(x, y, __builtin_fmaf(w, (float)(i + 1), y * p1), w);
          }
        }
      } else {
        double q = ipow_f64((double)lam, a.t_offset + row0 + tid);
        double step = lam;
#pragma unroll
        for (int k = 0; k < ilog2(NT); ++k) step *= step;
        for (int r = tid; r < L; r += NT) {
          const int64_t t = a.t_offset + row0 + r;
          float x = 0.0f, y = 0.0f;
          if (row0 + r < a.N) bwd_row_terms(lam, t + 1, q, x, y);
          const float w = x * p;
          sm.rt4[r + r / R] = make_float4(x, y, __builtin_fmaf(w, (float)(i + 1), y * p1), w);
          q *= step;
        }
      }
    }
    if (tid < DG) {
      sm.carry_s[tid] = cs;
      sm.gfin[tid] = cf;
    }
    __syncthreads();  // tables

    const int fin_i = rc == 0 && a.gfin != nullptr && li >= 0 && gr + li == left ? li : -1;

    // 16 rows per lane hold 128 registers of rows: there the forward sweep
    // takes the gy-only sums of rows 8-15 only, and rows 0-7 get a pass of
    // their own (sweep_gy) afterwards, so as not to hold 16 more registers
    // while every row is in flight.
    constexpr int kF0 = R <= 8 ? 0 : R / 2;
    float sl[VW], wl[VW], dq, qz[VW], ra[VW];
    sweep_fwd<kF0>(rv, rg, lam, g, fin_i, ds, sm, sl, wl, dq, qz, ra);
    // The launch epoch, first needed to publish (below).  Read here, once
    // every row has been consumed: loads complete in order, so waiting for it
    // earlier would have waited for every row (and holding it in a register
    // across the row loads would spill).
    const EpochErr eh = read_epoch_v(a.hdr);
    const unsigned epoch = eh.epoch;
    if constexpr (kF0 > 0) sweep_gy<kF0>(rg, g, fin_i, ds, sm, qz, ra);

    // Scans over the row groups of the wavefront, both directions: sl holds
    // the lane's forward total, ra its reverse total.
    group_scan<1, GW, VW, LPR>(sl, gw, sm.pw);
    group_scan_rev<1, GW, VW, LPR>(ra, gw, sm.pw);
    if (gw == GW - 1) {
#pragma unroll
      for (int j = 0; j < VW; ++j) sm.wt[wave][ds * VW + j] = sl[j];
    }
    if (gw == 0) {
#pragma unroll
      for (int j = 0; j < VW; ++j) sm.rt[wave][ds * VW + j] = ra[j];
    }
    float xin[VW], rin[VW];  // forward: state before the lane; reverse: g after the lane (wave-local)
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const float o = lane_shr<1, GW, LPR>(sl[j]);
      xin[j] = gw > 0 ? o : 0.0f;
      const float p = lane_shl<1, GW, LPR>(ra[j]);
      rin[j] = gw < GW - 1 ? p : 0.0f;
    }
    __syncthreads();

    // Reverse carry of the chunk by look-back over the chunks after it
    // (wavefront 0, first: later chunks wait on its inclusive word).
    const float mW = sm.pw[GW];
    float cg[DQ];
    bool poisoned = false;  // wavefront 0: the workspace's error word is set
    if (wave == 0) {
      const float mL = sm.pw[G];
      const unsigned tag_agg = tag_of(epoch, 0u), tag_inc = tag_of(epoch, 1u);
      u64* base = multi ? a.flags + (int64_t)stream * a.nchunk * DG : nullptr;
      float agg[DQ];
#pragma unroll
      for (int q = 0; q < DQ; ++q) {
        const int d = lane + 64 * q;
        agg[q] = 0.0f;
        cg[q] = 0.0f;
        if (d < DG) {
#pragma unroll
          for (int w = NW - 1; w >= 0; --w) agg[q] = __builtin_fmaf(mW, agg[q], sm.rt[w][d]);
          if (rc > 0 && chunk > 0) publish(base + (int64_t)rc * DG + d, tag_agg, agg[q]);
        }
      }
      // As in the forward: with the workspace's error word set, the carry is
      // NaN, nothing is waited for and nothing counts toward the epoch's
      // advance (dV, d(init) and the chunk's dlam partial, hence the head's
      // dlam, become NaN; every partial is still published, under the one
      // epoch all workgroups read, so the head sums do not wait either).
      poisoned = __builtin_amdgcn_readfirstlane(eh.err) != 0;
      if (poisoned) {
#pragma unroll
        for (int q = 0; q < DQ; ++q) cg[q] = __builtin_nanf("");
      } else if (rc > 0) {
        look_back<W, DG, DQ>(base, rc, tag_agg, tag_inc, mL, a.hdr, a.spin_limit, cg);
      }
#pragma unroll
      for (int q = 0; q < DQ; ++q) {
        const int d = lane + 64 * q;
        if (d < DG) {
          if (multi && chunk > 0) publish(base + (int64_t)rc * DG + d, tag_inc, __builtin_fmaf(mL, cg[q], agg[q]));
          sm.carry_g[d] = cg[q];
        }
      }
    }

    // s_in (true, from the saved chunk state) and g_out without the chunk's
    // carry; the carry-free part of the lane's dlam, and K per channel.
    // From here the chunk's dlam partial is summed in double (the lane's
    // channel terms, the wavefront and workgroup sums, the carry term): dlam
    // is often a small remainder of large terms of both signs, and in fp32
    // these sums lost most of its digits (B=45 H=1 N=1388 D=128 bf16, 8 M
    // terms for one head: relative error 1.9e-4 against 1.9e-6 in double,
    // and 1.3e-4 for the reference's own fp32 path; C2 unchanged, C4 and the
    // small grids 0.7-1.3% slower).  The lane's row sums (dq) stay fp32: in
    // double they took the registers of the narrow-group kernels.
    const float mg = sm.pw[g], mgw = sm.pw[gw];
    const float mr = sm.pw[G - 1 - g], mrw = sm.pw[GW - 1 - gw];
    const float rlr = (float)R * sm.pw[1];
    float gh0[VW];
    double dsum = dq;
    {
      float ew[VW], er[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        ew[j] = 0.0f;
        er[j] = 0.0f;
      }
      for (int w = 0; w < wave; ++w) {
#pragma unroll
        for (int j = 0; j < VW; ++j) ew[j] = __builtin_fmaf(mW, ew[j], sm.wt[w][ds * VW + j]);
      }
      for (int w = NW - 1; w > wave; --w) {
#pragma unroll
        for (int j = 0; j < VW; ++j) er[j] = __builtin_fmaf(mW, er[j], sm.rt[w][ds * VW + j]);
      }
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const float sin = __builtin_fmaf(mg, sm.carry_s[ds * VW + j], __builtin_fmaf(mgw, ew[j], xin[j]));
        gh0[j] = __builtin_fmaf(mrw, er[j], rin[j]);
        const float x = __builtin_fmaf(sin, rlr, lam * wl[j]);  // Q2 + s_in R lam^R
        dsum = __builtin_fma((double)gh0[j], (double)x, __builtin_fma((double)sin, (double)qz[j], dsum));
        sm.kq[g][ds * VW + j] = mr * x;
      }
    }
    dsum = wave_sum_f64(dsum);
    if (lane == 0) sm.red[wave] = dsum;
    __syncthreads();  // carry_g, kq, red

    // The chunk's dlam partial: the carry-free part plus carry * K.
    if (wave == 0) {
      double e = 0.0;
#pragma unroll
      for (int q = 0; q < DQ; ++q) {
        const int d = lane + 64 * q;
        if (d < DG) {
          double kc = 0.0;
#pragma unroll
          for (int r = 0; r < G; ++r) kc += (double)sm.kq[r][d];
          e = __builtin_fma((double)cg[q], kc, e);
        }
      }
      e = wave_sum_f64(e);
      if (lane == 0) {
        double sum = e;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += sm.red[w];
        publish(a.partial + (int64_t)rc * a.nstream + stream, tag_of(epoch, 0u), (float)sum);
      }
    }

    // Few streams: the first chunk of each stream counts, as soon as its
    // look-back is done (see the end of run()).
    if (a.per_stream && chunk == 0 && tid == 0 && !poisoned) count_done(a.hdr, (unsigned)a.nstream, epoch);

    // dV with the true carry.
    float gn[VW];
#pragma unroll
    for (int j = 0; j < VW; ++j) gn[j] = __builtin_fmaf(mr, sm.carry_g[ds * VW + j], gh0[j]);
    T* dp = static_cast<T*>(a.dv) + b * a.db + h * a.dh + grp * DG + row0 * a.dn + ((int64_t)gr * a.dn + ds * VW);
    sweep_dv(a, rg, lam, g, li, fin_i, ds, sm, dp, gn);
    if (a.dinit && row0 + gr == 0) {
#pragma unroll
      for (int j = 0; j < VW; ++j) a.dinit[c0 + ds * VW + j] = lam * gn[j];
    }

    // The workgroup with the largest item index of head h sums the head's
    // partials.  Every other item of the head has a smaller index, so it was
    // dispatched earlier and finishes without waiting on this workgroup.
    //
    // With many streams, the epoch advances once the H summing workgroups
    // and the last workgroup of each XCD have counted (ndone of them).  A summing
    // workgroup has seen a partial of every workgroup of its head, each
    // published after that workgroup read the epoch, so every workgroup of
    // the launch has read it.  The last ones of the XCDs matter when a
    // bounded wait gives up: a summing workgroup then counts without every
    // partial, and the advance still waits until each XCD has dispatched all
    // its workgroups.  A few atomics on the count, not one per stream: one
    // per stream put 768 on one word at B=48 N=512 H=16 D=64 bf16 (one chunk
    // per stream), 45.4 us against 29.4 us.  With few streams counting each
    // stream's first chunk before its dV pass (as the forward counts its
    // last chunks) takes the count off the launch's tail: 0.5-2% faster.
    if (rc == a.nchunk - 1 && b == a.B - 1 && grp == a.ng - 1)
      reduce_head(a, h, epoch, poisoned);
    else if (!a.per_stream && item + kXcds >= (int)gridDim.x && tid == 0 && !poisoned)
      count_done(a.hdr, (unsigned)a.ndone, epoch);
  }

  // dlam[h] = the sum of head h's chunk partials in double, in a fixed order
  // whatever the order in which they arrive (deterministic): wavefront 0
  // alone, each lane summing a strided subset (all its reads issued at
  // once), then a fixed butterfly across the lanes.
  __device__ static void reduce_head(const BwdArgs& a, int h, unsigned epoch, bool poisoned) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const unsigned tag = tag_of(epoch, 0u);
    const int n = (int)a.B * a.ng * a.nchunk;
    constexpr int K = 8;
    double acc = 0.0;
    for (int i0 = 0; i0 < n; i0 += 64 * K) {
      const u64* p[K];
      u64 w[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int idx = i0 + lane + 64 * k < n ? i0 + lane + 64 * k : n - 1;
        const int bg = (int)a.f_nchunk.div((uint32_t)idx), rc = idx - bg * a.nchunk;
        const int b = (int)a.f_ng.div((uint32_t)bg), grp = bg - b * a.ng;
        p[k] = a.partial + (int64_t)rc * a.nstream + ((int64_t)b * a.H + h) * a.ng + grp;
        w[k] = peek(p[k]);
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if (i0 + lane + 64 * k >= n) continue;
        for (int spin = 0; (unsigned)(w[k] >> 32) != tag; ++spin) {
          if (spin >= a.spin_limit) {  // give up: flag it, and the head's dlam becomes NaN
            __hip_atomic_store(a.hdr + HDR_ERROR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            w[k] = ((u64)tag << 32) | 0x7fc00000u;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          w[k] = peek(p[k]);
        }
        acc += (double)__uint_as_float((unsigned)w[k]);
      }
    }
    acc = wave_sum_f64(acc);
    if (lane == 0) {
      // Only the batch-slice kernels carry this (compiled into every kernel,
      // it cost one more VGPR, and five waves per SIMD, in the 4-row
      // narrow-group kernels and 1.2% at the B=8 N=4096 H=12 backward).
      if constexpr (SL) {
        if (a.slice + 1 < a.nslice) {
          a.dlam_slices[(int64_t)a.slice * a.H + h] = acc;  // the last slice adds it
        } else {
          double t = acc;
          if (a.slice > 0) {  // the earlier slices' sums in slice order, then this one's
            t = a.dlam_slices[h];
            for (int sl = 1; sl < a.slice; ++sl) t += a.dlam_slices[(int64_t)sl * a.H + h];
            t += acc;
          }
          a.dlam[h] = (float)t;
        }
      } else {
        a.dlam[h] = (float)acc;
      }
      if (!a.per_stream && !poisoned) count_done(a.hdr, (unsigned)a.ndone, epoch);
    }
  }
};

template <typename T, int LPR, int R, int NW, int W, int WPE, bool SL = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, 8))) void scan_bwd(BwdArgs a) {
  using CB = ChunkBwd<T, LPR, R, NW, W, SL>;
  __shared__ typename CB::Smem sm;
  CB::run(a, sm);
}

// --------------------------------------------------------------------------
// Sequential scan: one lane per (b,h,d) column, exact division.
// --------------------------------------------------------------------------
struct SeqArgs {
  const void* V;
  void* out;
  const float* lam;
  const float* init;
  float* fin;
  int64_t vs[4], os[4];
  int64_t B, H, N, D, t_offset;
};

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void scan_sequential(SeqArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.B * a.H * a.D) return;
  const int64_t d = idx % a.D;
  const int64_t bh = idx / a.D;
  const int64_t h = bh % a.H;
  const int64_t b = bh / a.H;
  const float lam = a.lam[h];
  const TI* vp = static_cast<const TI*>(a.V) + b * a.vs[0] + h * a.vs[1] + d * a.vs[3];
  TO* op = static_cast<TO*>(a.out) + b * a.os[0] + h * a.os[1] + d * a.os[3];
  float s = a.init ? a.init[idx] : 0.0f;
  for (int64_t t = 0; t < a.N; ++t) {
    s = lam * s + to_f32(vp[t * a.vs[2]]);
    op[t * a.os[2]] = from_f32<TO>(s / z_of(lam, a.t_offset + t));
  }
  if (a.fin) a.fin[idx] = s;
}

// --------------------------------------------------------------------------
// Decode step for the whole batch
// --------------------------------------------------------------------------
struct StepArgs {
  const float* lam;
  const float* s_in;
  const void* v;
  float* s_out;
  void* out;
  const int32_t* tpos;
  int64_t tpos_scalar;
  int64_t H, D, total;
  FastDiv f_D, f_H;  // division by D and H (the four-wide kernel)
};

template <typename TV, typename TO>
__global__ __launch_bounds__(256) void decay_step(StepArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.total) return;
  const int64_t bh = idx / a.D;
  const int64_t h = bh % a.H;
  const int64_t b = bh / a.H;
  // Load order and the unconditional position load as in decay_step4.
  const float lam = a.lam[h];
  int32_t tpv = *(a.tpos ? a.tpos + b : reinterpret_cast<const int32_t*>(a.lam));
  __builtin_amdgcn_sched_barrier(0);
  const float s = a.s_in[idx];
  const float v = to_f32(static_cast<const TV*>(a.v)[idx]);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" : "+v"(tpv)::"memory");
  const int64_t tp = a.tpos ? (int64_t)tpv : a.tpos_scalar;
  const float z = z_of_fast(lam, tp);
  const float ns = lam * s + v;  // two roundings (contraction is off)
  a.s_out[idx] = ns;
  static_cast<TO*>(a.out)[idx] = from_f32<TO>(ns / z);
}

// Four consecutive elements of T as floats / from floats (T: float, 16 bytes;
// bf16 or fp16, 8 bytes).  p must be aligned to the access size.
template <typename T>
__device__ __forceinline__ void load4(const T* p, float (&f)[4]) {
  if constexpr (sizeof(T) == 4) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
  } else {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    const uint4 u = make_uint4(x.x, x.y, 0u, 0u);
    float g[8];
    unpack16<T>(u, g);
    f[0] = g[0]; f[1] = g[1]; f[2] = g[2]; f[3] = g[3];
  }
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float (&f)[4]) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
  } else {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack2((T*)nullptr, f[0], f[1]), pack2((T*)nullptr, f[2], f[3]));
  }
}

// Decode step, four channels per thread (D % 4 == 0, aligned arrays).  The
// decay factor and the position are loaded first so the normaliser is
// computed while the state and v_t are in flight; z is evaluated once per
// thread instead of once per element.
template <typename TV, typename TO>
__global__ __launch_bounds__(256) void decay_step4(StepArgs a) {
  // 32-bit indices: the host launches this kernel only when total < 2^31.
  const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (idx >= (int)a.total) return;
  const int bh = (int)a.f_D.div((uint32_t)idx);
  const int b = (int)a.f_H.div((uint32_t)bh), h = bh - b * (int)a.H;
  // The decay factor and position first (z needs them first, and memory
  // operations complete in issue order), then the state and v.  The position
  // load is unconditional (a load under a branch is waited for at the branch
  // join, before the loads after it are issued): with no per-sequence
  // vector it reads the decay factor's bits and discards them.
  const float lam = a.lam[h];
  int32_t tpv = *(a.tpos ? a.tpos + b : reinterpret_cast<const int32_t*>(a.lam));
  __builtin_amdgcn_sched_barrier(0);  // keep those two loads ahead of the next two
  float s[4], v[4];
  load4<float>(a.s_in + idx, s);
  load4<TV>(static_cast<const TV*>(a.v) + idx, v);
  __builtin_amdgcn_sched_barrier(0);  // and all four issued before any is used
  asm volatile("" : "+v"(tpv)::"memory");  // no use of the position moves above the loads
  const int64_t tp = a.tpos ? (int64_t)tpv : a.tpos_scalar;
  const float z = z_of_fast(lam, tp);
  float ns[4], o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ns[j] = lam * s[j] + v[j];  // two roundings (contraction is off)
    o[j] = ns[j] / z;
  }
  store4<float>(a.s_out + idx, ns);
  store4<TO>(static_cast<TO*>(a.out) + idx, o);
}

__global__ __launch_bounds__(256) void zero_floats(float* p, int64_t n) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < n) p[idx] = 0.0f;
}

// Final state of an empty sequence: the initial state (or zeros).
__global__ __launch_bounds__(256) void copy_state(const float* init, float* fin, int64_t n) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < n) fin[idx] = init ? init[idx] : 0.0f;
}

// --------------------------------------------------------------------------
// Host side
// --------------------------------------------------------------------------
thread_local char g_err[512] = "";

// Poll limit of the bounded waits of the next launches (kdecay_debug_set_spin_limit);
// read and written atomically, since host threads may launch concurrently.
static int g_spin_limit = kSpinLimit;

int spin_limit() { return __atomic_load_n(&g_spin_limit, __ATOMIC_RELAXED); }

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: %s", what, hipGetErrorString(e));
  return 0;
}

int elem_size(int dt) { return dt == KDECAY_F32 ? 4 : dt == KDECAY_F64 ? 8 : 2; }
// Types of the training forward, the backward and the decode step.
bool dtype_ok(int dt) { return dt == KDECAY_F32 || dt == KDECAY_BF16 || dt == KDECAY_F16; }
// Types of the three forward scans: also float64 (V and out together).
bool fwd_dtype_ok(int dt) { return dtype_ok(dt) || dt == KDECAY_F64; }

// Launch shape of the chunked scan: a chunk holds NW * 64 lanes x R rows x
// 16 bytes = 64 KiB of input whatever the dtype and D, in 64 VGPRs per lane
// (half that for small grids; see chunk_shape).  Measured on MI355X at B=8
// N=4096 H=12 D=64 and B=1 N=65536 H=16 D=128 bf16 against R in {2..32}, NW
// in {2,4,8}: this is the fastest.
constexpr int kR = 16;
constexpr int kNW = 4;
constexpr int kWPE = 2;

// Compute units of the current device, cached per device (0 if unknown).
int cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (dev >= 0 && dev < 64 && __atomic_load_n(&cached[dev], __ATOMIC_RELAXED) > 0)
    return __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (dev >= 0 && dev < 64) __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
  return n;
}

// Workgroups of `kernel` that one compute unit holds at once (0 if unknown).
int workgroups_per_cu(const void* kernel, int block) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

// Channels of one stream: a head's row is split into groups of at most 128
// bytes (64 bf16/fp16 or 32 fp32 channels).
int64_t group_width(int v_dtype, int64_t D) {
  const int64_t full = 128 / elem_size(v_dtype);
  return D < full ? D : full;
}

// Channels of one backward stream: whole 256-byte rows (16 lanes per row,
// 256-row chunks) for 2-byte heads with a multiple of 128 channels when the
// grid is large and its chains short, else group_width.  Halves of 256-byte
// rows read by two streams each made the backward's two-round launches
// slower than its one-round ones.  Measured (bf16 D=128, same-box A/B on
// shared buffers, us, 128-byte / 256-byte groups): B=8 N=4096 H=12 (two
// rounds at 128 bytes; chains of 16 at 256 rows) 65.5 / 61.0; B=4 N=4096
// H=12 30.8 / 29.9; but B=1 N=65536 H=16 (chains of 256) 145.7 / 165.9 and
// B=8 N=1024 H=6 (a small grid, 128-row chunks at 128 bytes) 12.6 / 13.6.
constexpr int64_t kWideChain = 32;  // chunks of 256 rows per stream, at most
constexpr int64_t kWideGrid = 512;  // chunks of 256 rows in all, at least
int64_t bwd_group_width(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  if (elem_size(v_dtype) == 2 && D % 128 == 0) {
    const int64_t chain = (N + 255) / 256;
    if (chain <= kWideChain && chain * B * H * (D / 128) >= kWideGrid) return 128;
  }
  return group_width(v_dtype, D);
}

// Chunk shape: R rows per lane, NW wavefronts per workgroup; `six`: the
// 8-row grid built for six workgroups per compute unit (see chunk_shape).
struct ChunkShape {
  int R, NW;
  bool six = false;
};

int64_t chunk_rows(int v_dtype, int64_t D, ChunkShape c) {
  const int64_t vw = 16 / elem_size(v_dtype);
  const int64_t lpr = group_width(v_dtype, D) / vw;
  return c.NW * (64 / lpr) * c.R;
}

// Chunk shape of a problem: (kR, kNW), or (kRSmall, kNWSmall) when a
// (kR, kNW) grid would leave most of the device idle: at most kSmallGrid
// chunks, kSmallGrid2 with 2 chunks per stream (up to 1280 workgroups of 8
// rows; just above it they lose 13-19%, measured below) and kSmallGrid1 with
// 1 (the 16-row grid then needs no look-back at all, the 8-row one a chain of
// 2).
// Measured on MI355X (bf16, same-box A/B of the current kernels, 16 rows
// against 8, us; chunks at 16 rows): D=64 N=2048 B=8, 4 per stream: H=12
// (384) 11.62 / 10.58, H=14 (448) 11.87 / 11.96, H=16 (512) 12.46 / 12.99;
// N=1024 H=16, 2 per stream: B=16 (512) 13.56 /
// 12.72, B=19 (608) 15.19 / 14.84, B=20 (640) 15.48 / 15.40, B=21 (672)
// 15.64 / 18.69; D=128 N=1024 H=16 B=10 (640) 17.21 / 15.65, B=11 (704)
// 17.32 / 19.56; N=512 H=16, 1 per stream: B=8 (128) 7.42 / 7.16, B=10
// (160) 7.68 / 7.63, B=12 (192) 7.95 / 8.04, B=16 (256) 8.75 / 9.75, B=24
// (384) 10.18 / 11.53.  Long chains keep the 8-row grid (B=1 N=65536 H=2,
// 256 chunks: 26.42 / 20.41).  The rule uses the shape only, so
// kdecay_scan_workspace_bytes can apply it too.
constexpr int kRSmall = 8;
constexpr int kNWSmall = 4;
constexpr int64_t kSmallGrid = 416;
constexpr int64_t kSmallGrid2 = 640;
constexpr int64_t kSmallGrid1 = 160;

// Grids of 16-row chunks just above one resident round.  The 16-row kernels
// take 104-110 VGPRs, four workgroups per compute unit, 1024 on the 256 CUs
// of a gfx950 part; above that the launch runs a second, partial round, and
// at 1.5 rounds it lost 8-10 points of bandwidth against C2 and C4.  Held
// in 80 VGPRs (every 80-VGPR build of the 16-row kernel spilled 104-292
// bytes) the 8-row kernel runs six workgroups per compute unit, 1536 at
// once, so the same launch takes at most two full rounds of 256-row chunks,
// with a look-back window of 1 (the second round's chunks find their
// predecessors' inclusive words published in the first).  Measured (same-box
// A/B, us, 16-row kernel / 8-row six-per-CU window 1, all N=4096 H=12):
// bf16 D=128 B=6 (1152 chunks at 16 rows) 29.78 / 28.23, B=7 (1344) 35.19 /
// 31.67, B=8 (1536) 40.84 / 35.75 (61.6% -> 70.4% of 8 TB/s); fp32 D=64
// B=6 29.55 / 27.87, B=7 34.26 / 31.36, B=8 39.93 / 35.39 (63.0% -> 71.1%);
// bf16 D=64 B=11 (1056) 28.31 / 27.22, B=12 (1152) 28.94 / 29.45, B=13
// (1248) 31.01 / 31.72, B=14 (1344) 35.62 / 33.03, B=15 (1440) 37.45 /
// 35.41, B=16 (1536) 39.67 / 38.14.  Windows 2 and 4 were slower (bf16
// D=128 B=8: 37.7 and 37.4 us), and so was the 8-row grid outside this
// range: C2 (768, one round) 17.56 / 22.9 (window 2: 18.9), B=16 H=16 D=64
// (2048) 46.68 / 49.26, B=24 (2304) 57.8 / 60.1, C4 (4096) 91.5 / 169
// (window 4: 91.2), longer chains (16 chunks per stream: B=8 N=8192 H=12
// D=64 34.87 / 41.32, window 2 35.67).  So: 8 or fewer chunks per stream
// and 1280 < chunks <= 1536, or 1024 < chunks <= 1536 when a head has
// several channel groups (its streams then read strided halves of each row,
// where the 16-row kernel does worse).  Full 128-byte channel groups only:
// the 8-row kernel of narrower groups (more row groups per wavefront, a
// longer scan across them) spilled 36-60 bytes within 80 VGPRs.
constexpr int64_t kSixLo = 1280;
constexpr int64_t kSixLoGroups = 1024;
constexpr int64_t kSixHi = 1536;
constexpr int64_t kSixChain = 8;
// Heads of four or more channel groups (rows of 512 bytes or more, each
// stream reading every fourth 128-byte slice or sparser) keep the six-per-CU
// 8-row kernel at any grid of a full round or more, up to 32 chunks per
// stream: there the 16-row kernel loses 5-16 points.  Measured (same-box A/B
// on shared buffers, us, 16-row / 8-row six-per-CU, N=4096 unless given):
// fp64 D=64 B=8 H=12 (3072 chunks) 79.5 / 69.7 (63.3% -> 72.2% of 8 TB/s),
// B=16 181.9 / 151.5, B=6 58.0 / 53.0; bf16 D=256 B=8 H=12 80.9 / 70.3, fp32
// D=128 B=8 H=12 80.2 / 70.4; bf16 D=256 H=16: B=2 N=8192 (2048) 62.0 /
// 47.9, B=4 N=8192 (1024, chains of 16) 101.0 / 94.3, B=2 N=16384 (32 per
// stream) 97.6 / 91.0, B=8 N=2048 50.3 / 47.4, B=4 H=8 (1024) 29.2 / 25.2;
// eight groups: fp64 D=128 B=8 H=12 190.5 / 167.0, bf16 D=512 B=8 H=12 192.4
// / 168.7.  Not below a full round (bf16 D=256 B=2 H=12, 768 chunks: 18.7 /
// 21.2), not for longer chains (bf16 D=256 B=1 H=16: N=32768, 64 per stream,
// 96.4 / 117.7; N=65536 189.4 / 231.0), and not for fewer groups (three:
// bf16 D=192 B=8 H=12 60.7 / 60.4, fp64 D=48 B=12 H=12 89.4 / 90.4; two:
// fp32 D=64 B=16 H=12 70.1 / 72.4; one: bf16 D=64 B=32 H=12 71.9 / 76.3).
constexpr int64_t kSixWideGroups = 4;
constexpr int64_t kSixWideChain = 32;
constexpr int64_t kSixWideLo = 1024;

// Small grids of few, long streams: 512-row chunks of 8 wavefronts x 8 rows
// instead of 256-row chunks of 4 wavefronts, which halves the chain a carry
// crosses.  Measured (bf16 D=64, same-box A/B, us, 4 / 8 wavefronts, chain at
// 256 rows): B=1 N=65536 H=2 (256 per stream) 20.23 / 15.00, B=1 N=32768 H=6
// (128) 15.60 / 12.58, B=1 N=16384 H=6 (64) 10.26 / 9.74, B=1 N=16384 H=12
// (64) 12.32 / 11.92, B=2 N=16384 H=6 (64) 12.34 / 11.95; with 32 or fewer
// per stream the 4-wavefront chunks stay faster: B=1 N=8192 H=6 8.10 / 8.41,
// B=1 N=8192 H=16 9.03 / 9.38, B=2 N=8192 H=12 11.03 / 11.44, B=2 N=4096
// H=6 7.41 / 7.82.  (At the end-to-end model's layer shape, B=8 N=1024 H=6,
// the 4 x 8 chunk also beat 2 wavefronts x 8 rows, 4 x 4, 8 x 4 and 8 x 8:
// 6.49 against 6.61-7.43 us.)
constexpr int kNWLong = 8;
constexpr int64_t kLongChain = 64;

ChunkShape chunk_shape(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  const int64_t L = chunk_rows(v_dtype, D, ChunkShape{kR, kNW});
  const int64_t ng = D / group_width(v_dtype, D);
  const int64_t nstream = B * H * ng;
  const int64_t chain = (N + L - 1) / L;
  const int64_t grid = chain * nstream;
  const int64_t lim = chain == 1 ? kSmallGrid1 : chain == 2 ? kSmallGrid2 : kSmallGrid;
  const bool full = group_width(v_dtype, D) * elem_size(v_dtype) == 128;
  if (grid <= lim) {
    const int64_t chain8 = (N + L / 2 - 1) / (L / 2);  // chunks per stream at 8 rows per lane
    return full && chain8 >= kLongChain ? ChunkShape{kRSmall, kNWLong} : ChunkShape{kRSmall, kNWSmall};
  }
  if (full && chain <= kSixChain && grid > (ng > 1 ? kSixLoGroups : kSixLo) && grid <= kSixHi)
    return ChunkShape{kRSmall, kNWSmall, true};
  if (full && ng >= kSixWideGroups && chain <= kSixWideChain && grid >= kSixWideLo)
    return ChunkShape{kRSmall, kNWSmall, true};
  return ChunkShape{kR, kNW};
}

// Batch slices.  Heads of one full 128-byte channel group (bf16/fp16 D=64,
// fp32 D=32, fp64 D=16), a batch of at least 2, at most kSliceChain chunks
// of 512 rows per stream and more than one resident round of them
// (kSliceRound: four 16-row workgroups per CU on 256 CUs) run as that many
// launches over balanced slices of the batch, each one round at most of
// 512-row chunks: a launch of several rounds starts its later rounds only as
// the earlier ones finish, after their rows' full latency, where back-to-back
// launches overlap one's end with the next one's start.  Measured (bf16 D=64
// N=4096, same-box A/B, us, one launch / slices): H=12 B=11 27.7 / 26.5 (2),
// B=12 28.1 / 28.4 (2), B=13 29.9 / 29.6 (2), B=14 33.3 / 30.7 (2), B=16 38.4 / 35.1 (2), B=20 47.2 / 42.5 (2), B=24
// 57.7 / 52.3 (3), B=32 72.0 / 69.9 (4), B=48 110.4 / 105.6 (6), B=64 142.9 /
// 140.9 (8); H=16 B=10 32.1 / 30.0, B=12 38.0 / 34.6, B=16 46.5 / 44.2, B=24
// 71.6 / 66.4, B=40 120.4 / 110.8; N=2048 H=12 B=32 38.4 / 35.0, N=1024
// H=12 B=64 39.4 / 35.0, N=512 B=128 38.1 / 33.7; fp32 D=32 B=16 H=12 37.7 /
// 35.2.  Not for longer chains (N=8192 H=12 B=8, 16 per stream: 34.4 /
// 35.6) and not for heads of several groups, which the six-per-CU grid
// serves better (fp32 D=64 B=8 H=12 35.0 / 37.1 in two slices, fp64 D=64
// 70.0 / 75.4 in three).  Of the slice counts from the fewest that fit one
// round each to two more, the one with the fewest compute-unit rounds in all
// (n launches of ceil(B / n) batch elements, ceil(chunks / kSliceCUs)
// workgroups per CU each; ties to fewer launches): whole rounds of three or
// four workgroups per CU beat more, larger slices that leave CUs a workgroup
// short (B=64 H=12 in 7 slices of 9-10: 147.7, in 8 of 8: 140.9; B=48 in 5:
// 107.5, in 6: 105.6), and fewer launches win the ties (B=16 H=16 in 2: 44.2,
// in 3: 47.2; B=12 H=16 in 2: 34.6, in 3: 40.0).  Returns the number of
// launches (1: one for the whole batch); slice i holds batch elements
// [i B / n, (i+1) B / n).  At most kSliceMax launches, the range measured
// (each adds a launch's fixed cost): grids that need more run as one.  A grid
// of four rounds or more, whose one launch already spreads its round changes
// thin, is sliced only when the slices fill nine tenths of their workgroup
// slots (B=72 H=12: one launch 163.8, 8 slices of 864 chunks 167.6; B=80 in 8
// of 960: 181.7 / 172.6; B=56 in 7 of 768: 129.2 / 122.8).
constexpr int64_t kSliceRound = 1024;
constexpr int64_t kSliceCUs = 256;
constexpr int64_t kSliceChain = 8;
constexpr int64_t kSliceMax = 8;
int64_t fwd_slices(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  const int64_t DG = group_width(v_dtype, D);
  if (B < 2 || DG != D || DG * elem_size(v_dtype) != 128) return 1;
  const int64_t L = chunk_rows(v_dtype, D, ChunkShape{kR, kNW});
  const int64_t chain = (N + L - 1) / L;
  const int64_t per_b = H * chain;  // 512-row chunks of one batch element
  if (chain > kSliceChain || per_b > kSliceRound || B * per_b <= kSliceRound) return 1;
  const int64_t b_max = kSliceRound / per_b;
  const int64_t fewest = (B + b_max - 1) / b_max;
  if (fewest > kSliceMax) return 1;
  int64_t best = fewest, best_rounds = 0;
  for (int64_t n = fewest; n <= fewest + 2 && n <= B && n <= kSliceMax; ++n) {
    const int64_t rounds = n * (((B + n - 1) / n * per_b + kSliceCUs - 1) / kSliceCUs);
    if (n == fewest || rounds < best_rounds) best = n, best_rounds = rounds;
  }
  const int64_t chunks = (B + best - 1) / best * per_b;
  const int64_t slots = (chunks + kSliceCUs - 1) / kSliceCUs * kSliceCUs;
  if (B * per_b >= 4 * kSliceRound && 10 * chunks < 9 * slots) return 1;
  return best;
}

// Head dims of the chunked kernels: 16, 32, or any multiple of a full
// 128-byte channel group (64 bf16/fp16 or 32 fp32 channels); a head is then
// D / group_width independent streams.  (A group of 16 or 32 channels takes
// 2 or 4 lanes per row; other widths would not divide a wavefront.)
bool head_dim_ok(int v_dtype, int64_t D) {
  const int64_t full = 128 / elem_size(v_dtype);
  return D == 16 || D == 32 || (D > 0 && D % full == 0);
}

template <typename TI, typename TO, int DG, int R = kR, int NW = kNW, int WPE = kWPE>
int launch_chunked(const ScanArgs& a, int64_t grid, hipStream_t s, bool six = false) {
  constexpr int VW = 16 / (int)sizeof(TI);
  constexpr int LPR = DG / VW;
  // Small grids are latency-bound: there the per-row normaliser table uses
  // the unrolled, branch-free power (B=8 N=1024 H=6 D=64 bf16: 7.07 -> 6.85
  // us); for large grids the loop form is cheaper (B=8 N=4096 H=12 D=64:
  // 18.36 vs 18.74 us with the unrolled one).  Same values either way.
  constexpr bool FZ = R == kRSmall && NW == kNWSmall;
  if constexpr (FZ) {
    if constexpr (LPR == 8) {  // full 128-byte channel groups
      if (six) {  // chunk_shape's 8-row grid, six workgroups per CU (two rounds at most, except wide heads)
        hipLaunchKernelGGL((scan_chunked<TI, TO, LPR, R, NW, 1, 6, FZ, false>), dim3((unsigned)grid), dim3(NW * 64), 0,
                           s, a);
        return hip_check("scan_chunked launch");
      }
    }
    // Small grids run in one round.  Long chains of few streams want a wide
    // window: a chunk then folds the aggregates of its predecessors, each
    // published as soon as that chunk is scanned, instead of waiting for their
    // inclusive prefixes hop by hop.  Measured (bf16 D=64, same-box A/B,
    // window 4 / 8 / 16): B=1 N=32768 H=6 (128 chunks per stream) 27.97 /
    // 19.44 / 15.75 us; B=1 N=16384 H=12 (64) 17.45 / 13.81 / 12.49 us; B=1
    // N=8192 H=6 (32) 11.33 / 9.40 / 8.65 us; B=2 N=4096 H=12 (16) 8.99 /
    // 8.23 / -; B=8 N=1024 H=6 (4 chunks per stream) 7.00 / 6.89 / -.
    // Stores throttled (THR) when more than two workgroups share a CU on
    // average: B=8 N=2048 H=12 D=64 (768 workgroups) 10.68 -> 10.52 us, B=4
    // N=4096 H=12 11.10 -> 10.80 us; at 1.5 per CU (B=8 N=2048 H=6) it was
    // 0.5% slower, and no change at fewer.
    const bool thr = grid > 2 * (int64_t)cu_count();
    auto* const k = a.nchunk > 16 ? (thr ? scan_chunked<TI, TO, LPR, R, NW, 16, WPE, FZ, true>
                                         : scan_chunked<TI, TO, LPR, R, NW, 16, WPE, FZ, false>)
                  : a.nchunk > 4  ? (thr ? scan_chunked<TI, TO, LPR, R, NW, 8, WPE, FZ, true>
                                         : scan_chunked<TI, TO, LPR, R, NW, 8, WPE, FZ, false>)
                                  : (thr ? scan_chunked<TI, TO, LPR, R, NW, kW, WPE, FZ, true>
                                         : scan_chunked<TI, TO, LPR, R, NW, kW, WPE, FZ, false>);
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(NW * 64), 0, s, a);
  } else {
    // The resident grid throttles its stores (three workgroups per CU share
    // the CU's memory path; THR): B=8 N=4096 H=12 D=64 bf16 18.13 -> 17.70
    // us, same-box A/B, identical outputs.  Launches in several rounds
    // measured no gain (B=1 N=65536 H=16 D=128 +0.3%).
    auto* const one_round = scan_chunked<TI, TO, LPR, R, NW, kW, WPE, FZ, true>;
    auto* const rounds = scan_chunked<TI, TO, LPR, R, NW, kWRounds, WPE, FZ, false>;
    // Several rounds with at most 16 resident chunk rows per stream (resident
    // workgroups over streams): a window of 1 (each chunk waits for its
    // predecessor's inclusive word, mostly already published in an earlier
    // round).  Measured (bf16, 4 workgroups per CU, same-box A/B, window 1
    // against 2): B=8 N=8192 H=12 D=64 (10.7 rows per round) 35.1 / 39.3 us,
    // B=5 N=16384 H=16 D=64 (12.8) 56.3 / 60.9, B=2 N=65536 H=16 D=128 (16)
    // 179.1 / 187.1, B=4 N=16384 H=16 D=128 (8) 96.1 / 98.3; with more rows
    // per round window 2 wins: B=7 N=16384 H=8 D=64 (18.3) 43.4 / 42.1, B=4
    // N=16384 H=12 D=64 (21.3) 39.6 / 35.3, B=1 N=65536 H=16 D=128 (32) 106 /
    // 91.5.
    auto* const rounds1 = scan_chunked<TI, TO, LPR, R, NW, 1, WPE, FZ, false>;
    static const int per_cu = workgroups_per_cu(reinterpret_cast<const void*>(one_round), NW * 64);
    const int64_t resident = (int64_t)per_cu * cu_count();
    if (resident > 0 && grid > resident)
      hipLaunchKernelGGL(resident <= 16 * (int64_t)a.nstream ? rounds1 : rounds, dim3((unsigned)grid), dim3(NW * 64), 0,
                         s, a);
    else
      hipLaunchKernelGGL(one_round, dim3((unsigned)grid), dim3(NW * 64), 0, s, a);
  }
  return hip_check("scan_chunked launch");
}

// The long-chain small grids of chunk_shape: 8 wavefronts x 8 rows, window 16.
template <typename TI, typename TO, int DG>
int launch_long(const ScanArgs& a, int64_t grid, hipStream_t s) {
  constexpr int LPR = DG / (16 / (int)sizeof(TI));
  hipLaunchKernelGGL((scan_chunked<TI, TO, LPR, kRSmall, kNWLong, 16, kWPE, true, false>), dim3((unsigned)grid),
                     dim3(kNWLong * 64), 0, s, a);
  return hip_check("scan_chunked launch");
}

// DG: channels per stream (group_width); R, NW: the chunk shape (chunk_shape).
template <typename TI, typename TO, int R, int NW>
int dispatch_dg_r(const ScanArgs& a, int64_t DG, int64_t grid, hipStream_t s, bool six) {
  switch (DG) {
    case 16: return launch_chunked<TI, TO, 16, R, NW>(a, grid, s, six);
    case 32:  // a 128-byte group of fp32, or half of one (bf16/fp16); fp64 groups have 16
      if constexpr (sizeof(TI) <= 4) return launch_chunked<TI, TO, 32, R, NW>(a, grid, s, six);
      break;
    case 64:
      if constexpr (sizeof(TI) == 2) return launch_chunked<TI, TO, 64, R, NW>(a, grid, s, six);
      break;
  }
  return fail(KDECAY_ESHAPE, "unsupported channel group %lld", (long long)DG);
}

template <typename TI, typename TO>
int dispatch_dg(const ScanArgs& a, int64_t DG, int64_t grid, hipStream_t s, ChunkShape c) {
  if (c.R == kRSmall && c.NW == kNWLong) {
    // Long chains only (window 16, fewer workgroups than twice the CUs: no throttle), full groups.
    constexpr int kFull = 128 / (int)sizeof(TI);
    if (DG == kFull) return launch_long<TI, TO, kFull>(a, grid, s);
    return fail(KDECAY_ESHAPE, "unsupported channel group %lld", (long long)DG);
  }
  if (c.R == kRSmall && c.NW == kNWSmall) return dispatch_dg_r<TI, TO, kRSmall, kNWSmall>(a, DG, grid, s, c.six);
  return dispatch_dg_r<TI, TO, kR, kNW>(a, DG, grid, s, false);
}

// Launch shape of the backward scan: 4 wavefronts; 16 rows per lane (512-row
// chunks of a 128-byte channel group: V and gy of the chunk in registers, at
// most 168 VGPRs for 3 workgroups per CU), or 4 rows per lane when the
// 16-row grid would leave most of the device idle.  The look-back window is
// 4 when the whole grid is resident, else 2 (as for the forward).
constexpr int kRB = 16;
constexpr int kRBSmall = 4;
constexpr int kNWB = 4;
constexpr int64_t kBwdSmallGrid = 256;
// Streams up to which every stream's first chunk counts toward the epoch's
// advance (ChunkBwd::run).  Measured (bf16, same-box A/B, per stream / per
// head and XCD, us): D=64 B=8 N=1024 H=6 (48 streams) 11.13 / 11.48; B=8
// N=4096 H=12 (96) 28.77 / 29.17; B=12 N=2048 H=16 (192) 29.31 / 29.61;
// B=16 N=2048 H=16 (256) 40.68 / 40.86; B=16 N=1024 H=16 (256) 23.96 /
// 23.21; B=24 N=1024 H=16 (384) 37.23 / 29.21.
constexpr int64_t kBwdPerStreamCount = 192;
constexpr int64_t kBwdShortChainGrid = 384;

// 4 rows per lane when the 16-row grid has at most kBwdSmallGrid chunks, so
// that the 4-row grid (4x the workgroups) still runs in one round, or at most
// kBwdShortChainGrid chunks with chains of at most 4 (the 4-row grid then
// takes 1.5 rounds of chains at most 16 chunks long); longer chains in
// several rounds run with a narrow window and lose.  Measured (same-box A/B,
// bf16, 4 rows vs 16 rows, us): D=64 B=8 N=1024 H=6 (96 chunks at 16 rows)
// 11.3 / 16.2; B=8 N=2048 H=10 (320, 4 per stream) 19.1 / 21.1; B=8 N=2048
// H=12 (384, 4) 20.1 / 21.8; B=12 N=1024 H=16 (384, 2) 20.5 / 22.6; B=4
// N=4096 H=12 (384, 8) 22.9 / 22.2; B=2 N=8192 H=12 (384, 16) 31.7 / 22.3;
// B=8 N=2048 H=14 (448, 4) 23.2 / 22.9; D=32 B=8 N=4096 H=12 (384, 4)
// 24.5 / 28.6; D=32 B=8 N=4096 H=16 (512, 4) 32.4 / 29.8.
// 8 rows per lane (256-row chunks, 128 VGPRs, four workgroups per CU
// instead of three) for heads of two or more 128-byte channel groups, when
// the 16-row grid runs more than one round and has at least 48 streams.
// Measured (same-box A/B on shared buffers, each variant's own saved states,
// us, 16 / 8 rows; N=4096 H=12 unless given): fp32 D=64 B=5 (960 chunks of
// 512 rows) 42.4 / 39.4, B=6 50.9 / 46.9, B=8 (two rounds) 64.7 / 60.1, B=16
// 109.6 / 106.8; fp32 D=128 B=4 66.8 / 59.0, B=8 113.4 / 102.5; fp32 D=64
// H=16 B=2 N=16384 78.3 / 74.4, B=24 N=1024 58.4 / 57.4; fp32 D=128 B=1 H=16
// N=65536 (64 streams) 280.6 / 263.9 (71.8% -> 76.3% of 8 TB/s); bf16 D=128
// B=2 H=16 N=32768 (64 streams) 146.0 / 140.9, bf16 D=256 B=1 N=65536 (48)
// 217.1 / 208.2.  Not in one round (fp32 D=64 B=4, 768 chunks: 30.1 /
// 33.7), not for one-group heads (fp32 D=32 B=12 H=12 46.8 / 48.6, bf16 D=64
// B=16 H=12 60.8 / 62.5, C2 27.2 / 35.6) and not for fewer streams (bf16
// D=128 B=1 H=16 N=65536, 32 streams: 145.7 / 147.5; fp16 147.0 / 147.9).
// Whole 256-byte rows keep 16 rows (bwd_group_width).
constexpr int kRBMid = 8;
constexpr int64_t kBwdOneRound = 768;  // resident 16-row chunks on 256 CUs
constexpr int64_t kBwdMidStreams = 48;
// Also 8 rows per lane for 128-byte groups when the 16-row grid has more
// than 192 and at most 512 chunks: the 8-row grid then runs in one round of
// at most 1024 (four per CU) where the 16-row one fills at most two thirds
// of its 768 slots and the 4-row one pays chains four times as long.
// Measured (bf16 D=64, same-box A/B on shared buffers, us, current choice /
// 8 rows): 16-row grids B=4 N=4096 H=12 (384 chunks) 19.16 / 17.23, B=7
// N=2048 H=16 (448) 19.77 / 19.01, B=4 N=4096 H=16 (512) 21.18 / 19.98, B=2
// N=8192 H=16 (512) 22.49 / 21.23, B=1 N=16384 H=12 (384, chains of 32)
// 20.1 / 19.48, bf16 D=128 B=2 N=4096 H=12 (384) 19.91 / 17.26; 4-row grids
// B=8 N=2048 H=12 (384, chains of 4) 21.23 / 16.71, B=6 N=2048 H=12 (288)
// 19.22 / 15.35, B=1 N=8192 H=16 (256) 19.78 / 14.59, B=4 N=4096 H=8 (256)
// 15.00 / 14.38, B=8 N=2048 H=8 (256) 14.00 / 13.85.  Not at 192 chunks or
// fewer (B=8 N=1024 H=12, 192: 12.30 / 13.00; H=6, the end-to-end model's
// layer: 10.26 / 10.90) nor at a full 16-row round (B=5 N=4096 H=16, 640:
// 24.87 / 31.00; B=3 N=8192 H=16, 768: 27.44 / 33.19).
constexpr int64_t kBwdMidLo = 192;
constexpr int64_t kBwdMidHi = 512;
int bwd_rows_per_lane(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  const int64_t vw = 16 / elem_size(v_dtype);
  const int64_t DG = bwd_group_width(B, H, N, D, v_dtype);
  const int64_t L = kNWB * (64 / (DG / vw)) * kRB;
  const int64_t nstream = B * H * (D / DG);
  const int64_t chain = (N + L - 1) / L;
  const int64_t grid = chain * nstream;
  const bool g128 = DG * elem_size(v_dtype) == 128;
  if (g128 && grid > kBwdMidLo && grid <= kBwdMidHi) return kRBMid;
  if (grid <= kBwdSmallGrid || (grid <= kBwdShortChainGrid && chain <= 4)) return kRBSmall;
  if (g128 && D / DG >= 2 && grid > kBwdOneRound && nstream >= kBwdMidStreams) return kRBMid;
  return kRB;
}

int64_t bwd_chunk_rows(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  const int64_t vw = 16 / elem_size(v_dtype);
  const int64_t lpr = bwd_group_width(B, H, N, D, v_dtype) / vw;
  return kNWB * (64 / lpr) * bwd_rows_per_lane(B, H, N, D, v_dtype);
}

template <typename T, int DG>
int launch_bwd(const BwdArgs& a, int64_t grid, int R, hipStream_t s) {
  constexpr int VW = 16 / (int)sizeof(T);
  constexpr int LPR = DG / VW;
  if (R == kRB) {
    // Batch slices (bwd_slices): one full round each, chains of at most 8.
    if (a.nslice > 1) {
      if constexpr (LPR == 8) {
        hipLaunchKernelGGL((scan_bwd<T, LPR, kRB, kNWB, kW, 3, true>), dim3((unsigned)grid), dim3(kNWB * 64), 0, s, a);
        return hip_check("scan_bwd launch");
      } else {
        return fail(KDECAY_ESHAPE, "no batch-slice backward kernel for %d-channel groups", DG);
      }
    }
    // One round: window 4, or 8 for chains of more than 8 chunks (a window
    // of 16 does not fit beside 16 rows per lane without spilling); several
    // rounds: 2.
    auto* const one_round = scan_bwd<T, LPR, kRB, kNWB, kW, 3>;
    static const int per_cu = workgroups_per_cu(reinterpret_cast<const void*>(one_round), kNWB * 64);
    const int64_t resident = (int64_t)per_cu * cu_count();
    auto* const k = resident > 0 && grid > resident ? scan_bwd<T, LPR, kRB, kNWB, kWRounds, 3>
                    : a.nchunk > 8                  ? scan_bwd<T, LPR, kRB, kNWB, 8, 3>
                                                    : one_round;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kNWB * 64), 0, s, a);
  } else if (R == kRBMid) {
    // 256-row chunks (bwd_rows_per_lane): one round at four workgroups per CU
    // (window 4, or 8 for chains of more than 8), or several.
    if constexpr (LPR == 8) {
      auto* const w4 = scan_bwd<T, LPR, kRBMid, kNWB, kW, 4>;
      static const int per_cu = workgroups_per_cu(reinterpret_cast<const void*>(w4), kNWB * 64);
      const int64_t resident = (int64_t)per_cu * cu_count();
      auto* const k = resident > 0 && grid > resident ? scan_bwd<T, LPR, kRBMid, kNWB, kWRounds, 4>
                      : a.nchunk > 8                  ? scan_bwd<T, LPR, kRBMid, kNWB, 8, 4>
                                                      : w4;
      hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kNWB * 64), 0, s, a);
    } else {
      return fail(KDECAY_ESHAPE, "no 8-row backward kernel for %d-channel groups", DG);
    }
  } else if constexpr (LPR >= 16) {
    // Whole 256-byte rows only on large grids (bwd_group_width), which take
    // 16 rows per lane.
    return fail(KDECAY_ESHAPE, "no small-grid kernel for %d-channel groups", DG);
  } else {
    // Small grids: by chain length when the grid is resident, as for the
    // forward's small grids.  Measured (bf16 D=64, same-box A/B, window 2 /
    // 4 / 8): B=8 N=1024 H=6 (8 chunks per stream) 12.13 / 11.73 / 11.94 us;
    // B=2 N=4096 H=12 (32) 19.65 / 15.73 / 14.90 us; B=1 N=8192 H=6 (64)
    // 28.11 / 20.45 / 16.34 us.  The window-16 kernel holds 32 registers of
    // look-back words: within 128 VGPRs (4 waves per SIMD) it spilled 20-24
    // bytes, so it is built for 3 waves per SIMD (B=1 N=16384 H=6 20.1 ->
    // 18.4 us, B=1 N=65536 H=2 43.1 -> 39.7 us, same-box A/B).
    auto* const w4 = scan_bwd<T, LPR, kRBSmall, kNWB, 4, 4>;
    static const int per_cu = workgroups_per_cu(reinterpret_cast<const void*>(w4), kNWB * 64);
    const int64_t resident = (int64_t)per_cu * cu_count();
    auto* const k = resident > 0 && grid > resident ? scan_bwd<T, LPR, kRBSmall, kNWB, kWRounds, 4>
                    : a.nchunk > 32                 ? scan_bwd<T, LPR, kRBSmall, kNWB, 16, 3>
                    : a.nchunk > 8                  ? scan_bwd<T, LPR, kRBSmall, kNWB, 8, 4>
                                                    : w4;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kNWB * 64), 0, s, a);
  }
  return hip_check("scan_bwd launch");
}

template <typename T>
int dispatch_bwd(const BwdArgs& a, int64_t DG, int64_t grid, int R, hipStream_t s) {
  switch (DG) {
    case 16: return launch_bwd<T, 16>(a, grid, R, s);
    case 32: return launch_bwd<T, 32>(a, grid, R, s);
    case 64:
      if constexpr (sizeof(T) == 2) return launch_bwd<T, 64>(a, grid, R, s);
      break;
    case 128:  // whole 256-byte rows (bwd_group_width): 16-row chunks only
      if constexpr (sizeof(T) == 2) return launch_bwd<T, 128>(a, grid, R, s);
      break;
  }
  return fail(KDECAY_ESHAPE, "unsupported channel group %lld", (long long)DG);
}

template <typename TI, typename TO>
int launch_seq(const SeqArgs& a, hipStream_t s) {
  const int64_t n = a.B * a.H * a.D;
  hipLaunchKernelGGL((scan_sequential<TI, TO>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
  return hip_check("scan_sequential launch");
}

// The four-wide kernel when D is a multiple of 4 and every array is aligned
// to its 4-element access, else one thread per element.
template <typename TV, typename TO>
int launch_step(const StepArgs& a, hipStream_t s) {
  const bool vec = a.total < (int64_t)1 << 31 && a.D % 4 == 0 && (uintptr_t)a.s_in % 16 == 0 && (uintptr_t)a.s_out % 16 == 0 &&
                   (uintptr_t)a.v % (4 * sizeof(TV)) == 0 && (uintptr_t)a.out % (4 * sizeof(TO)) == 0;
  if (vec) {
    const int64_t nq = a.total / 4;
    hipLaunchKernelGGL((decay_step4<TV, TO>), dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((decay_step<TV, TO>), dim3((unsigned)((a.total + 255) / 256)), dim3(256), 0, s, a);
  }
  return hip_check("decay_step launch");
}

// Common argument checks of the two scan entry points.
int check_scan_args(const void* V, int v_dtype, const int64_t* v_strides, const void* out, int out_dtype,
                    const int64_t* out_strides, const float* lam, int64_t B, int64_t H, int64_t N,
                    int64_t D) {
  if (B < 0 || H < 0 || N < 0 || D < 0) return fail(KDECAY_EINVAL, "negative size");
  if (!fwd_dtype_ok(v_dtype) || !fwd_dtype_ok(out_dtype))
    return fail(KDECAY_EDTYPE, "unknown dtype code (v=%d out=%d)", v_dtype, out_dtype);
  if (out_dtype != v_dtype && (out_dtype != KDECAY_F32 || v_dtype == KDECAY_F64))
    return fail(KDECAY_EDTYPE, "out dtype must equal V's dtype or be F32 (F64: V's dtype only)");
  if (B * H * N * D == 0) return 0;
  if (!V || !out || !lam || !v_strides || !out_strides) return fail(KDECAY_EINVAL, "null pointer argument");
  return 0;
}

int empty_final_state(const float* init, float* fin, int64_t n, hipStream_t s) {
  if (!fin || n == 0) return 0;
  hipLaunchKernelGGL(copy_state, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, init, fin, n);
  return hip_check("copy_state launch");
}

}  // namespace kd

// Look-back workspace of kdecay_scan_fwd_noalloc: a fixed array in the code
// object's device memory, so that entry point allocates nothing.  Each GPU the
// library is loaded on holds its own copy, at its own address, until the
// process ends.  It has no initialiser, so the loader zero-fills it when the
// code object is loaded on a device (a zeroed workspace is what the epoch
// protocol starts from); the library never clears it again.  On the host this
// name is only a stand-in for the symbol, not a device address: host code
// uses the address hipGetSymbolAddress returns for the current device
// (scratch_of_current_device), never `scratch` itself.
static __device__ __align__(256) unsigned char scratch[KDECAY_NOALLOC_WORKSPACE_BYTES];

namespace kd {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device (null until set up)

// Device address of the current device's scratch array.  The first call on a
// device looks the address up (hipGetSymbolAddress, with that device current);
// nothing is launched or recorded for it, so a first call under stream
// capture records only the scan.  Later calls find the epoch protocol's state
// in place.
int scratch_of_current_device(void** p) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(KDECAY_EINVAL, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail((int)e, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    if (!ptr) return fail(KDECAY_EINVAL, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr[dev] = ptr;
  }
  *p = g_scratch_ptr[dev];
  return 0;
}

}  // namespace kd

using namespace kd;

extern "C" {

const char* kdecay_version(void) { return "kdecay 0.1.0 gfx950"; }

const char* kdecay_last_error_string(void) { return g_err; }

int kdecay_debug_set_spin_limit(int polls) {
  const int previous =
      __atomic_exchange_n(&g_spin_limit, polls > 0 && polls < kSpinLimit ? polls : kSpinLimit, __ATOMIC_RELAXED);
  return previous == kSpinLimit ? 0 : previous;
}

uint32_t kdecay_debug_fastdiv(uint32_t n, uint32_t d, int want_mod) {
  if (d == 0) return 0;
  const FastDiv f = make_fastdiv(d);
  return want_mod ? f.mod(n) : f.div(n);
}

size_t kdecay_scan_workspace_bytes(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  if (B <= 0 || H <= 0 || N <= 0 || !fwd_dtype_ok(v_dtype) || !head_dim_ok(v_dtype, D)) return 0;
  const int64_t n = fwd_slices(B, H, N, D, v_dtype);
  // Batch slices run one after another on the workspace: the largest one's.
  const int64_t Bs = (B + n - 1) / n;
  const int64_t L = chunk_rows(v_dtype, D, n > 1 ? ChunkShape{kR, kNW} : chunk_shape(B, H, N, D, v_dtype));
  const int64_t nchunk = (N + L - 1) / L;
  if (nchunk <= 1) return 0;
  return kHeaderBytes + (size_t)(Bs * H * nchunk * D) * sizeof(u64);
}

static int scan_fwd_impl(const void* V, int v_dtype, const int64_t* v_strides, void* out, int out_dtype,
                         const int64_t* out_strides, const float* lam, const float* init_state,
                         float* final_state, int64_t B, int64_t H, int64_t N, int64_t D, int64_t t_offset,
                         void* workspace, size_t workspace_bytes, float* states, void* stream) {
  int rc = check_scan_args(V, v_dtype, v_strides, out, out_dtype, out_strides, lam, B, H, N, D);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B * H * D == 0) return 0;
  if (N == 0) return empty_final_state(init_state, final_state, B * H * D, s);
  if (!head_dim_ok(v_dtype, D))
    return fail(KDECAY_ESHAPE, "head dim D=%lld is not 16, 32 or a multiple of %d", (long long)D,
                128 / elem_size(v_dtype));

  const int64_t vw_in = 16 / elem_size(v_dtype);
  const int64_t vw_out = 16 / elem_size(out_dtype);
  if (v_strides[3] != 1 || out_strides[3] != 1) return fail(KDECAY_ELAYOUT, "channel (d) stride must be 1");
  if (((uintptr_t)V & 15u) || ((uintptr_t)out & 15u)) return fail(KDECAY_ELAYOUT, "V and out must be 16-byte aligned");
  const int64_t sizes[3] = {B, H, N};
  for (int k = 0; k < 3; ++k) {  // a size-1 dim's stride is never used
    if (sizes[k] > 1 && (v_strides[k] % vw_in || out_strides[k] % vw_out))
      return fail(KDECAY_ELAYOUT, "stride %d is not a multiple of 16 bytes", k);
  }

  const int64_t DG = group_width(v_dtype, D);
  {
    const int64_t L = chunk_rows(v_dtype, D, chunk_shape(B, H, N, D, v_dtype));
    const int64_t nchunk = (N + L - 1) / L, nstream = B * H * (D / DG), grid = nchunk * nstream;
    if (grid > 0x7fffffffLL || nchunk > 0x7fffffffLL || nstream > 0x7fffffffLL)
      return fail(KDECAY_EINVAL, "problem too large (%lld chunks)", (long long)grid);
  }
  const size_t need = kdecay_scan_workspace_bytes(B, H, N, D, v_dtype);
  if (need && (!workspace || workspace_bytes < need))
    return fail(KDECAY_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
  if (need && ((uintptr_t)workspace & 255u)) return fail(KDECAY_EWORKSPACE, "workspace must be 256-byte aligned");

  // The training forward's saved states follow the whole batch's backward
  // chunks, and batch 0's workgroups write the per-row terms once.
  const int64_t state_rows = bwd_chunk_rows(B, H, N, D, v_dtype);
  const int64_t nsaved = (N + state_rows - 1) / state_rows;
  float* const saved = nsaved > 1 ? states : nullptr;
  float2* const rowtab = saved ? reinterpret_cast<float2*>(saved + B * H * D * nsaved) : nullptr;
  const int64_t nslice = fwd_slices(B, H, N, D, v_dtype);
  for (int64_t i = 0; i < nslice; ++i) {
    const int64_t b0 = B * i / nslice, Bs = B * (i + 1) / nslice - b0;
    const ChunkShape shape = nslice > 1 ? ChunkShape{kR, kNW} : chunk_shape(B, H, N, D, v_dtype);
    const int64_t L = chunk_rows(v_dtype, D, shape);
    const int64_t nchunk = (N + L - 1) / L;
    const int64_t nstream = Bs * H * (D / DG);
    const int64_t grid = nchunk * nstream;
    const bool multi = nchunk > 1;

    ScanArgs a;
    a.V = static_cast<const char*>(V) + b0 * v_strides[0] * elem_size(v_dtype);
    a.out = static_cast<char*>(out) + b0 * out_strides[0] * elem_size(out_dtype);
    a.lam = lam;
    a.init = init_state ? init_state + b0 * H * D : nullptr;
    a.fin = final_state ? final_state + b0 * H * D : nullptr;
    a.vb = v_strides[0];
    a.vh = v_strides[1];
    a.vn = v_strides[2];
    a.ob = out_strides[0];
    a.oh = out_strides[1];
    a.on = out_strides[2];
    a.H = H;
    a.N = N;
    a.t_offset = t_offset;
    a.D = D;
    a.ng = (int)(D / DG);
    a.nchunk = (int)nchunk;
    a.nstream = (int)nstream;
    a.f_nstream = make_fastdiv((uint32_t)nstream);
    a.f_ng = make_fastdiv((uint32_t)a.ng);
    a.f_H = make_fastdiv((uint32_t)H);
    a.hdr = multi ? static_cast<unsigned*>(workspace) : nullptr;
    a.spin_limit = spin_limit();
    a.flags = multi ? reinterpret_cast<u64*>(static_cast<char*>(workspace) + kHeaderBytes) : nullptr;
    a.state_rows = state_rows;
    a.nsaved = nsaved;
    a.states = saved ? saved + b0 * H * D * nsaved : nullptr;
    a.rowtab = i == 0 ? rowtab : nullptr;

    if (v_dtype == KDECAY_F32)
      rc = dispatch_dg<float, float>(a, DG, grid, s, shape);
    else if (v_dtype == KDECAY_F64)
      rc = dispatch_dg<double, double>(a, DG, grid, s, shape);
    else if (v_dtype == KDECAY_BF16)
      rc = out_dtype == KDECAY_BF16 ? dispatch_dg<__bf16, __bf16>(a, DG, grid, s, shape)
                                    : dispatch_dg<__bf16, float>(a, DG, grid, s, shape);
    else
      rc = out_dtype == KDECAY_F16 ? dispatch_dg<_Float16, _Float16>(a, DG, grid, s, shape)
                                   : dispatch_dg<_Float16, float>(a, DG, grid, s, shape);
    if (rc) return rc;
  }
  return 0;
}

int kdecay_scan_fwd(const void* V, int v_dtype, const int64_t* v_strides, void* out, int out_dtype,
                    const int64_t* out_strides, const float* lam, const float* init_state,
                    float* final_state, int64_t B, int64_t H, int64_t N, int64_t D, int64_t t_offset,
                    void* workspace, size_t workspace_bytes, void* stream) {
  return scan_fwd_impl(V, v_dtype, v_strides, out, out_dtype, out_strides, lam, init_state, final_state, B, H, N, D,
                       t_offset, workspace, workspace_bytes, nullptr, stream);
}

int kdecay_scan_fwd_noalloc(const void* V, int v_dtype, const int64_t* v_strides, void* out, int out_dtype,
                            const int64_t* out_strides, const float* lam, const float* init_state,
                            float* final_state, int64_t B, int64_t H, int64_t N, int64_t D, int64_t t_offset,
                            void* stream) {
  const int rc = check_scan_args(V, v_dtype, v_strides, out, out_dtype, out_strides, lam, B, H, N, D);
  if (rc) return rc;
  const size_t need = kdecay_scan_workspace_bytes(B, H, N, D, v_dtype);
  if (need > KDECAY_NOALLOC_WORKSPACE_BYTES)
    return fail(KDECAY_EWORKSPACE,
                "kdecay_scan_fwd_noalloc: this shape needs %zu bytes of look-back workspace, more than the "
                "library's fixed %zu-byte device array; use kdecay_scan_fwd with a workspace",
                need, (size_t)KDECAY_NOALLOC_WORKSPACE_BYTES);
  void* ws = nullptr;
  if (need) {
    const int e = scratch_of_current_device(&ws);
    if (e) return e;
  }
  return scan_fwd_impl(V, v_dtype, v_strides, out, out_dtype, out_strides, lam, init_state, final_state, B, H, N, D,
                       t_offset, ws, need ? (size_t)KDECAY_NOALLOC_WORKSPACE_BYTES : 0, nullptr, stream);
}

size_t kdecay_scan_saved_states_floats(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  if (B <= 0 || H <= 0 || N <= 0 || !dtype_ok(v_dtype) || !head_dim_ok(v_dtype, D)) return 0;
  const int64_t Lb = bwd_chunk_rows(B, H, N, D, v_dtype);
  const int64_t nsaved = (N + Lb - 1) / Lb;
  if (nsaved <= 1) return 0;
  // The states at the backward's chunk starts, then the backward's two terms
  // of every row of every head (ScanArgs::rowtab).
  return (size_t)(B * H * D * nsaved + 2 * H * N);
}

int kdecay_scan_fwd_train(const void* V, int v_dtype, const int64_t* v_strides, void* out, int out_dtype,
                          const int64_t* out_strides, const float* lam, const float* init_state,
                          float* final_state, float* states, size_t states_floats, int64_t B, int64_t H,
                          int64_t N, int64_t D, int64_t t_offset, void* workspace, size_t workspace_bytes,
                          void* stream) {
  // The backward that reads these states takes no float64 (dtype_ok).
  if (!dtype_ok(v_dtype) || !dtype_ok(out_dtype))
    return fail(KDECAY_EDTYPE, "training forward: dtype code (v=%d out=%d) not F32/BF16/F16", v_dtype, out_dtype);
  const size_t need = kdecay_scan_saved_states_floats(B, H, N, D, v_dtype);
  if (need && (!states || states_floats < need))
    return fail(KDECAY_EINVAL, "states buffer of %zu floats required, %zu given", need, states_floats);
  return scan_fwd_impl(V, v_dtype, v_strides, out, out_dtype, out_strides, lam, init_state, final_state, B, H, N, D,
                       t_offset, workspace, workspace_bytes, states, stream);
}

// Backward batch slices.  Heads of one full 128-byte channel group on 512-row
// chunks, at most kSliceChain per stream, whose grid is exactly two or three
// resident rounds (kBwdOneRound chunks each) divided evenly by the batch: one
// launch per round-sized slice of the batch, in order on the stream, each
// slice's dlam sums kept in double in the workspace and added, in slice
// order, by the last slice.  Measured (bf16 D=64 N=4096, same-box, us, one
// launch / slices): H=12 B=16 59.25 / 55.28 (2), B=24 88.0 / 83.3 (3); H=16
// B=12 59.8 / 55.9 (2).  Not in other slicings: slices of part of a round
// (B=20 H=12 in 2: 72.5 / 75.0; B=12 H=12 in 2: 44.7 / 51.0) or four rounds
// (B=32 H=12 in 4: 109.2 / 112.0).  Returns the number of launches.
int64_t bwd_slices(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  const int64_t DG = bwd_group_width(B, H, N, D, v_dtype);
  if (B < 2 || DG != D || DG * elem_size(v_dtype) != 128 || bwd_rows_per_lane(B, H, N, D, v_dtype) != kRB) return 1;
  const int64_t chain = (N + bwd_chunk_rows(B, H, N, D, v_dtype) - 1) / bwd_chunk_rows(B, H, N, D, v_dtype);
  const int64_t grid = B * H * chain;
  if (chain > kSliceChain) return 1;
  for (int64_t n = 2; n <= 3; ++n)
    if (B % n == 0 && grid == n * kBwdOneRound) return n;
  return 1;
}

size_t kdecay_scan_bwd_workspace_bytes(int64_t B, int64_t H, int64_t N, int64_t D, int v_dtype) {
  if (B <= 0 || H <= 0 || N <= 0 || !dtype_ok(v_dtype) || !head_dim_ok(v_dtype, D)) return 0;
  const int64_t n = bwd_slices(B, H, N, D, v_dtype);
  const int64_t Bs = B / n;  // slices run one after another on the workspace
  const int64_t Lb = bwd_chunk_rows(B, H, N, D, v_dtype);
  const int64_t nchunk = (N + Lb - 1) / Lb;
  const size_t flags = nchunk > 1 ? (size_t)(Bs * H * nchunk * D) * sizeof(u64) : 0;
  const int64_t nstream = Bs * H * (D / bwd_group_width(B, H, N, D, v_dtype));
  const size_t partial = ((size_t)(nstream * nchunk) * sizeof(u64) + 255) & ~(size_t)255;
  const size_t sums = n > 1 ? ((size_t)((n - 1) * H) * sizeof(double) + 255) & ~(size_t)255 : 0;
  return kHeaderBytes + flags + partial + sums;
}

int kdecay_scan_bwd(const void* V, int v_dtype, const int64_t* v_strides, const void* gy,
                    const int64_t* gy_strides, void* dV, const int64_t* dv_strides, const float* lam,
                    const float* init_state, const float* states, const float* g_final, float* dlam,
                    float* d_init, int64_t B, int64_t H, int64_t N, int64_t D, int64_t t_offset,
                    void* workspace, size_t workspace_bytes, void* stream) {
  if (B < 0 || H < 0 || N < 0 || D < 0) return fail(KDECAY_EINVAL, "negative size");
  if (!dtype_ok(v_dtype)) return fail(KDECAY_EDTYPE, "unknown dtype code %d", v_dtype);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B * H * D == 0) return 0;
  if (!lam || !dlam) return fail(KDECAY_EINVAL, "null pointer argument");
  if (N == 0) {  // no rows: the gradients are the final-state gradient passed through
    hipLaunchKernelGGL(copy_state, dim3((unsigned)((B * H * D + 255) / 256)), dim3(256), 0, s, g_final,
                       d_init, d_init ? B * H * D : 0);
    int e = hip_check("copy_state launch");
    if (e) return e;
    hipLaunchKernelGGL(zero_floats, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, s, dlam, H);
    return hip_check("zero_floats launch");
  }
  if (!V || !gy || !dV || !v_strides || !gy_strides || !dv_strides) return fail(KDECAY_EINVAL, "null pointer argument");
  if (!head_dim_ok(v_dtype, D))
    return fail(KDECAY_ESHAPE, "head dim D=%lld is not 16, 32 or a multiple of %d", (long long)D,
                128 / elem_size(v_dtype));
  const int64_t vw = 16 / elem_size(v_dtype);
  if (v_strides[3] != 1 || gy_strides[3] != 1 || dv_strides[3] != 1)
    return fail(KDECAY_ELAYOUT, "channel (d) stride must be 1");
  if (((uintptr_t)V & 15u) || ((uintptr_t)gy & 15u) || ((uintptr_t)dV & 15u))
    return fail(KDECAY_ELAYOUT, "V, gy and dV must be 16-byte aligned");
  const int64_t sizes[3] = {B, H, N};
  for (int k = 0; k < 3; ++k) {
    if (sizes[k] > 1 && (v_strides[k] % vw || gy_strides[k] % vw || dv_strides[k] % vw))
      return fail(KDECAY_ELAYOUT, "stride %d is not a multiple of 16 bytes", k);
  }
  const int RB = bwd_rows_per_lane(B, H, N, D, v_dtype);
  const int64_t Lb = bwd_chunk_rows(B, H, N, D, v_dtype);
  const int64_t nchunk = (N + Lb - 1) / Lb;
  const int64_t DG = bwd_group_width(B, H, N, D, v_dtype);
  const int64_t nstream = B * H * (D / DG);
  const int64_t grid = nchunk * nstream;
  if (grid > 0x7fffffffLL) return fail(KDECAY_EINVAL, "problem too large (%lld chunks)", (long long)grid);
  // The kernel addresses a chunk's rows of V and gy by 32-bit offsets.
  const int64_t es = elem_size(v_dtype);
  if (v_strides[2] < 0 || gy_strides[2] < 0) return fail(KDECAY_ELAYOUT, "negative row stride");
  if (N > 1 && (Lb * v_strides[2] * es > 0x7fffffffLL || Lb * gy_strides[2] * es > 0x7fffffffLL))
    return fail(KDECAY_ELAYOUT, "row stride too large (%lld rows of a chunk exceed 2^31 bytes)", (long long)Lb);
  if (nchunk > 1 && !states) return fail(KDECAY_EINVAL, "saved states (kdecay_scan_fwd_train) required");
  const size_t need = kdecay_scan_bwd_workspace_bytes(B, H, N, D, v_dtype);
  if (!workspace || workspace_bytes < need)
    return fail(KDECAY_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
  if ((uintptr_t)workspace & 255u) return fail(KDECAY_EWORKSPACE, "workspace must be 256-byte aligned");

  // Batch slices (bwd_slices): the saved states keep the whole batch's
  // layout (nchunk per stream, then the per-row terms after all of them).
  const int64_t nslice = bwd_slices(B, H, N, D, v_dtype);
  const int64_t Bs = B / nslice;
  const int64_t nstream_s = Bs * H * (D / DG), grid_s = nchunk * nstream_s;
  const size_t flag_bytes = nchunk > 1 ? (size_t)(Bs * H * nchunk * D) * sizeof(u64) : 0;
  const size_t partial_bytes = ((size_t)(nstream_s * nchunk) * sizeof(u64) + 255) & ~(size_t)255;
  for (int64_t i = 0; i < nslice; ++i) {
    const int64_t b0 = i * Bs;
    BwdArgs a;
    a.V = static_cast<const char*>(V) + b0 * v_strides[0] * es;
    a.gy = static_cast<const char*>(gy) + b0 * gy_strides[0] * es;
    a.dv = static_cast<char*>(dV) + b0 * dv_strides[0] * es;
    a.lam = lam;
    a.init = init_state ? init_state + b0 * H * D : nullptr;
    a.states = states ? states + b0 * H * D * nchunk : nullptr;
    a.gfin = g_final ? g_final + b0 * H * D : nullptr;
    a.dinit = d_init ? d_init + b0 * H * D : nullptr;
    a.dlam = dlam;
    a.vb = v_strides[0];
    a.vh = v_strides[1];
    a.vn = v_strides[2];
    a.gb = gy_strides[0];
    a.gh = gy_strides[1];
    a.gn = gy_strides[2];
    a.db = dv_strides[0];
    a.dh = dv_strides[1];
    a.dn = dv_strides[2];
    a.B = Bs;
    a.H = H;
    a.N = N;
    a.t_offset = t_offset;
    a.D = D;
    a.ng = (int)(D / DG);
    a.nchunk = (int)nchunk;
    a.nstream = (int)nstream_s;
    a.nsaved = nchunk;
    a.rowtab = nchunk > 1 ? reinterpret_cast<const float2*>(states + B * H * D * nchunk) : nullptr;
    a.f_nstream = make_fastdiv((uint32_t)nstream_s);
    a.f_ng = make_fastdiv((uint32_t)a.ng);
    a.f_H = make_fastdiv((uint32_t)H);
    a.f_nchunk = make_fastdiv((uint32_t)nchunk);
    a.hdr = static_cast<unsigned*>(workspace);
    a.spin_limit = spin_limit();
    // Workgroups that count toward the epoch's advance: the H that sum a
    // head's partials (the last row of items, chunk 0, is unrotated: item
    // (nchunk-1)*nstream + stream with b = B-1 and the last channel group) and
    // the last of each XCD, each counted once.
    a.per_stream = nstream_s <= kBwdPerStreamCount;
    a.ndone = (int)H;
    for (int64_t item = grid_s > kXcds ? grid_s - kXcds : 0; item < grid_s; ++item) {
      const int64_t rc = item / nstream_s, stream = item - rc * nstream_s;
      const int64_t bh = stream / a.ng, grp = stream - bh * a.ng;
      const bool sums = rc == nchunk - 1 && bh / H == Bs - 1 && grp == a.ng - 1;
      if (!sums) ++a.ndone;
    }
    a.flags = nchunk > 1 ? reinterpret_cast<u64*>(static_cast<char*>(workspace) + kHeaderBytes) : nullptr;
    a.partial = reinterpret_cast<u64*>(static_cast<char*>(workspace) + kHeaderBytes + flag_bytes);
    a.slice = (int)i;
    a.nslice = (int)nslice;
    a.dlam_slices = reinterpret_cast<double*>(static_cast<char*>(workspace) + kHeaderBytes + flag_bytes + partial_bytes);
    int e;
    if (v_dtype == KDECAY_F32)
      e = dispatch_bwd<float>(a, DG, grid_s, RB, s);
    else if (v_dtype == KDECAY_BF16)
      e = dispatch_bwd<__bf16>(a, DG, grid_s, RB, s);
    else
      e = dispatch_bwd<_Float16>(a, DG, grid_s, RB, s);
    if (e) return e;
  }
  return 0;
}

int kdecay_scan_fwd_sequential(const void* V, int v_dtype, const int64_t* v_strides, void* out,
                               int out_dtype, const int64_t* out_strides, const float* lam,
                               const float* init_state, float* final_state, int64_t B, int64_t H,
                               int64_t N, int64_t D, int64_t t_offset, void* stream) {
  int rc = check_scan_args(V, v_dtype, v_strides, out, out_dtype, out_strides, lam, B, H, N, D);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B * H * D == 0) return 0;
  if (N == 0) return empty_final_state(init_state, final_state, B * H * D, s);
  if (D > 1024) return fail(KDECAY_ESHAPE, "head dim D=%lld > 1024", (long long)D);
  if ((B * H * D + 255) / 256 > 0x7fffffffLL) return fail(KDECAY_EINVAL, "problem too large");
  SeqArgs a;
  a.V = V;
  a.out = out;
  a.lam = lam;
  a.init = init_state;
  a.fin = final_state;
  for (int k = 0; k < 4; ++k) {
    a.vs[k] = v_strides[k];
    a.os[k] = out_strides[k];
  }
  a.B = B;
  a.H = H;
  a.N = N;
  a.D = D;
  a.t_offset = t_offset;
  if (v_dtype == KDECAY_F32) return launch_seq<float, float>(a, s);
  if (v_dtype == KDECAY_F64) return launch_seq<double, double>(a, s);
  if (v_dtype == KDECAY_BF16) {
    if (out_dtype == KDECAY_BF16) return launch_seq<__bf16, __bf16>(a, s);
    return launch_seq<__bf16, float>(a, s);
  }
  if (out_dtype == KDECAY_F16) return launch_seq<_Float16, _Float16>(a, s);
  return launch_seq<_Float16, float>(a, s);
}

int kdecay_step(const float* lam, const float* state_in, const void* v_t, int v_dtype, float* state_out,
                void* out, int out_dtype, const int32_t* t_pos, int64_t t_pos_scalar, int64_t B, int64_t H,
                int64_t D, void* stream) {
  if (B < 0 || H < 0 || D < 0) return fail(KDECAY_EINVAL, "negative size");
  if (!dtype_ok(v_dtype) || !dtype_ok(out_dtype))
    return fail(KDECAY_EDTYPE, "unknown dtype code (v=%d out=%d)", v_dtype, out_dtype);
  const int64_t total = B * H * D;
  if (total == 0) return 0;
  if (!lam || !state_in || !v_t || !state_out || !out) return fail(KDECAY_EINVAL, "null pointer argument");
  if ((total + 255) / 256 > 0x7fffffffLL) return fail(KDECAY_EINVAL, "problem too large");
  StepArgs a;
  a.lam = lam;
  a.s_in = state_in;
  a.v = v_t;
  a.s_out = state_out;
  a.out = out;
  a.tpos = t_pos;
  a.tpos_scalar = t_pos_scalar;
  a.H = H;
  a.D = D;
  a.total = total;
  a.f_D = make_fastdiv((uint32_t)D);
  a.f_H = make_fastdiv((uint32_t)H);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (v_dtype * 3 + out_dtype) {
    case KDECAY_F32 * 3 + KDECAY_F32: return launch_step<float, float>(a, s);
    case KDECAY_F32 * 3 + KDECAY_BF16: return launch_step<float, __bf16>(a, s);
    case KDECAY_F32 * 3 + KDECAY_F16: return launch_step<float, _Float16>(a, s);
    case KDECAY_BF16 * 3 + KDECAY_F32: return launch_step<__bf16, float>(a, s);
    case KDECAY_BF16 * 3 + KDECAY_BF16: return launch_step<__bf16, __bf16>(a, s);
    case KDECAY_BF16 * 3 + KDECAY_F16: return launch_step<__bf16, _Float16>(a, s);
    case KDECAY_F16 * 3 + KDECAY_F32: return launch_step<_Float16, float>(a, s);
    case KDECAY_F16 * 3 + KDECAY_BF16: return launch_step<_Float16, __bf16>(a, s);
    default: return launch_step<_Float16, _Float16>(a, s);
  }
}

}  // extern "C"
