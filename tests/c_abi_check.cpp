// A native C++ caller of libkdecay.so through include/kdecay.h alone (no Python,
// no torch): the full-sequence scan of a bf16 [B,H,N,D] tensor against a
// double-precision CPU recurrence, the decode step bit for bit against the same
// two float roundings on the CPU (attention.py:344-360), and a rejected
// argument.  Built by tests/c_abi_build.py; run by tests/test_gpu_scan.py.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "kdecay.h"

#define CHECK_HIP(x)                                                            \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      return 1;                                                                 \
    }                                                                           \
  } while (0)

static uint16_t to_bf16(float f) {  // round to nearest even
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float from_bf16(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

int main() {
  const int64_t B = 2, H = 3, N = 1500, D = 64, n = B * H * N * D;
  const float lam[3] = {0.9f, 0.999f, 0.5f};
  std::vector<uint16_t> hv(n);
  uint32_t s = 7u;
  for (int64_t i = 0; i < n; ++i) {
    s = s * 1664525u + 1013904223u;
    hv[i] = to_bf16(((s >> 9) & 0xffffu) / 32768.0f - 1.0f);
  }
  void *V, *Y, *ws;
  float *dlam, *fin;
  CHECK_HIP(hipMalloc(&V, n * 2));
  CHECK_HIP(hipMalloc(&Y, n * 2));
  CHECK_HIP(hipMalloc(&dlam, sizeof(lam)));
  CHECK_HIP(hipMalloc(&fin, B * H * D * 4));
  CHECK_HIP(hipMemcpy(V, hv.data(), n * 2, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dlam, lam, sizeof(lam), hipMemcpyHostToDevice));
  const int64_t st[4] = {H * N * D, N * D, D, 1};
  const size_t wsb = kdecay_scan_workspace_bytes(B, H, N, D, KDECAY_BF16);
  CHECK_HIP(hipMalloc(&ws, wsb ? wsb : 256));
  CHECK_HIP(hipMemset(ws, 0, wsb ? wsb : 256));
  int rc = kdecay_scan_fwd(V, KDECAY_BF16, st, Y, KDECAY_BF16, st, dlam, nullptr, fin, B, H, N, D, 0, ws, wsb,
                           nullptr);
  if (rc) {
    std::printf("kdecay_scan_fwd returned %d: %s\n", rc, kdecay_last_error_string());
    return 1;
  }
  CHECK_HIP(hipDeviceSynchronize());
  std::vector<uint16_t> hy(n);
  std::vector<float> hfin(B * H * D);
  CHECK_HIP(hipMemcpy(hy.data(), Y, n * 2, hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(hfin.data(), fin, B * H * D * 4, hipMemcpyDeviceToHost));
  double max_abs = 0.0, max_fin = 0.0;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t d = 0; d < D; ++d) {
        double state = 0.0;
        const double l = lam[h];
        for (int64_t t = 0; t < N; ++t) {
          const int64_t i = ((b * H + h) * N + t) * D + d;
          state = l * state + from_bf16(hv[i]);
          const double z = (1.0 - std::pow(l, (double)(t + 1))) / ((1.0 - l) + 1e-6);
          max_abs = std::fmax(max_abs, std::fabs(from_bf16(hy[i]) - state / z));
        }
        const double f = hfin[(b * H + h) * D + d];
        max_fin = std::fmax(max_fin, std::fabs(f - state) / std::fmax(1.0, std::fabs(state)));
      }
  if (!(max_abs <= 2e-2 && max_fin <= 1e-4)) {
    std::printf("scan mismatch: max_abs %.3e final-state %.3e\n", max_abs, max_fin);
    return 1;
  }

  // Decode step from the final state: the reference's two roundings, bit for bit.
  std::vector<uint16_t> hvt(B * H * D);
  for (auto& x : hvt) {
    s = s * 1664525u + 1013904223u;
    x = to_bf16(((s >> 9) & 0xffffu) / 32768.0f - 1.0f);
  }
  void* vt;
  float *sout, *out;
  CHECK_HIP(hipMalloc(&vt, B * H * D * 2));
  CHECK_HIP(hipMalloc(&sout, B * H * D * 4));
  CHECK_HIP(hipMalloc(&out, B * H * D * 4));
  CHECK_HIP(hipMemcpy(vt, hvt.data(), B * H * D * 2, hipMemcpyHostToDevice));
  rc = kdecay_step(dlam, fin, vt, KDECAY_BF16, sout, out, KDECAY_F32, nullptr, N, B, H, D, nullptr);
  if (rc) {
    std::printf("kdecay_step returned %d: %s\n", rc, kdecay_last_error_string());
    return 1;
  }
  CHECK_HIP(hipDeviceSynchronize());
  std::vector<float> hs(B * H * D);
  CHECK_HIP(hipMemcpy(hs.data(), sout, B * H * D * 4, hipMemcpyDeviceToHost));
  for (int64_t i = 0; i < B * H * D; ++i) {
    volatile float p = lam[(i / D) % H] * hfin[i];  // rounded product, then the rounded sum
    const float ns = p + from_bf16(hvt[i]);
    if (std::memcmp(&ns, &hs[i], 4) != 0) {
      std::printf("step state differs at %lld: %.9g vs %.9g\n", (long long)i, ns, hs[i]);
      return 1;
    }
  }

  // A rejected argument: negative code, nothing launched, a message.
  rc = kdecay_scan_fwd(V, 7, st, Y, KDECAY_BF16, st, dlam, nullptr, nullptr, B, H, N, D, 0, ws, wsb, nullptr);
  if (rc >= 0 || std::strlen(kdecay_last_error_string()) == 0) {
    std::printf("bad dtype was not rejected (rc %d)\n", rc);
    return 1;
  }
  std::printf("c_abi_check OK: %s; scan max_abs %.3e, final state %.3e, step state bit-identical\n",
              kdecay_version(), max_abs, max_fin);
  return 0;
}
