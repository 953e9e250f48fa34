/*
 * decay_oracle.c — plain-C oracle of Kilat's global-decay scan.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (and bench.py's CPU baseline
 * leg) as a checker; the product never links it.
 *
 * An independent restatement of /root/reference/src/kilat/arc/
 * triton_ops.py:232-247 and attention.py:344-360, written from the
 * arithmetic rather than from torch: every fp32 operation is one IEEE
 * rounding (built with -ffp-contract=off, SSE math), and lam^e follows the
 * value torch's pow(tensor, int) produces for a small tensor: lam for e=1,
 * lam*lam for e=2, (lam*lam)*lam for e=3, else the double power rounded to
 * float.  Agreement bit for bit with the torch restatement
 * (oracle/decay_oracle.py) pins both.
 *
 * Also an fp64 O(N^2) brute force of the defining sum
 *     y_i = sum_{j<=i} lam^(i-j) V_j / z_i
 * that shares no loop structure with the recurrence.
 */
#include <math.h>
#include <stdint.h>

static float pow_like_torch(float x, int64_t e) {
  if (e == 1) return x;
  if (e == 2) return x * x;
  if (e == 3) return (x * x) * x;
  if (e == 0) return 1.0f;
  return (float)pow((double)x, (double)e);
}

static float z_of(float lam, int64_t t) {
  const float num = 1.0f - pow_like_torch(lam, t + 1);
  const float den = (1.0f - lam) + 1e-6f;
  return num / den;
}

/* V, out: contiguous [B,H,N,D] fp32.  init, fin: [B,H,D] or NULL. */
void oracle_scan_f32(const float* V, const float* lam, float* out, const float* init, float* fin,
                     int64_t B, int64_t H, int64_t N, int64_t D, int64_t t_offset) {
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      const float l = lam[h];
      for (int64_t d = 0; d < D; ++d) {
        float s = init ? init[(b * H + h) * D + d] : 0.0f;
        const float* v = V + ((b * H + h) * N) * D + d;
        float* y = out + ((b * H + h) * N) * D + d;
        for (int64_t t = 0; t < N; ++t) {
          const float p = l * s;
          s = p + v[t * D];
          y[t * D] = s / z_of(l, t_offset + t);
        }
        if (fin) fin[(b * H + h) * D + d] = s;
      }
    }
  }
}

/* One decode step; t_pos: [B] or NULL (then t_pos_scalar for every row). */
void oracle_step_f32(const float* lam, const float* s_in, const float* v, float* s_out, float* out,
                     const int64_t* t_pos, int64_t t_pos_scalar, int64_t B, int64_t H, int64_t D) {
  for (int64_t b = 0; b < B; ++b) {
    const int64_t tp = t_pos ? t_pos[b] : t_pos_scalar;
    for (int64_t h = 0; h < H; ++h) {
      const float l = lam[h];
      const float z = z_of(l, tp);
      for (int64_t d = 0; d < D; ++d) {
        const int64_t i = (b * H + h) * D + d;
        const float p = l * s_in[i];
        const float ns = p + v[i];
        s_out[i] = ns;
        out[i] = ns / z;
      }
    }
  }
}

/* fp64 dense brute force of the definition, V/out contiguous [B,H,N,D]. */
void oracle_bruteforce_f64(const double* V, const double* lam, double* out, int64_t B, int64_t H, int64_t N,
                           int64_t D) {
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      const double l = lam[h];
      const double* v = V + ((b * H + h) * N) * D;
      double* y = out + ((b * H + h) * N) * D;
      for (int64_t i = 0; i < N; ++i) {
        const double z = (1.0 - pow(l, (double)(i + 1))) / (1.0 - l + 1e-6);
        for (int64_t d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int64_t j = 0; j <= i; ++j) acc += pow(l, (double)(i - j)) * v[j * D + d];
          y[i * D + d] = acc / z;
        }
      }
    }
  }
}
