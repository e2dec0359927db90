/*
 * Independent fp64 brute-force FlashMLP (test infrastructure only).
 *
 * Plain loops over the definitions, no shared code with the torch restatement:
 *   Z[h,b,e] = sum_d X[h,b,d] W1[h,d,e]           flashmlp.py:674
 *   Hh = act(Z)                                     flashmlp.py:676-683
 *   O[h,b,d] = sum_e Hh[h,b,e] W2[h,e,d]            flashmlp.py:685
 *   dH = dO W2^T, dZ = dH * act'(Z), dX = dZ W1^T, dW1 = X^T dZ, dW2 = Hh^T dO
 *                                                   README.md:57-61, flashmlp.py:705-721
 * act codes: 0 linear, 1 silu, 2 leaky_relu (slope 0.01, derivative 0.01 at 0 as autograd),
 * 3 sigmoid. All arrays row-major doubles with the reference's shapes.
 */
#include <math.h>
#include <stdlib.h>

static double sigm(double z) { return 1.0 / (1.0 + exp(-z)); }

static double act_f(double z, int act) {
  switch (act) {
    case 1: return z * sigm(z);
    case 2: return z > 0 ? z : 0.01 * z;
    case 3: return sigm(z);
    default: return z;
  }
}

static double act_d(double z, int act) {
  switch (act) {
    case 1: { double s = sigm(z); return s * (1.0 + z * (1.0 - s)); }
    case 2: return z > 0 ? 1.0 : 0.01;
    case 3: { double s = sigm(z); return s * (1.0 - s); }
    default: return 1.0;
  }
}

void brute_fwd(const double* X, const double* W1, const double* W2, double* O, int H, int B, int D, int E, int act) {
  for (int h = 0; h < H; ++h)
    for (int b = 0; b < B; ++b)
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int e = 0; e < E; ++e) {
          double z = 0.0;
          for (int k = 0; k < D; ++k) z += X[((long)h * B + b) * D + k] * W1[((long)h * D + k) * E + e];
          acc += act_f(z, act) * W2[((long)h * E + e) * D + d];
        }
        O[((long)h * B + b) * D + d] = acc;
      }
}

void brute_bwd(const double* X, const double* W1, const double* W2, const double* dO, double* dX, double* dW1,
               double* dW2, int H, int B, int D, int E, int act) {
  double* Z = (double*)malloc(sizeof(double) * (size_t)B * E);
  double* dZ = (double*)malloc(sizeof(double) * (size_t)B * E);
  for (int h = 0; h < H; ++h) {
    const double* x = X + (long)h * B * D;
    const double* w1 = W1 + (long)h * D * E;
    const double* w2 = W2 + (long)h * E * D;
    const double* go = dO + (long)h * B * D;
    for (int b = 0; b < B; ++b)
      for (int e = 0; e < E; ++e) {
        double z = 0.0, dh = 0.0;
        for (int k = 0; k < D; ++k) {
          z += x[(long)b * D + k] * w1[(long)k * E + e];
          dh += go[(long)b * D + k] * w2[(long)e * D + k];
        }
        Z[(long)b * E + e] = z;
        dZ[(long)b * E + e] = dh * act_d(z, act);
      }
    for (int b = 0; b < B; ++b)
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int e = 0; e < E; ++e) acc += dZ[(long)b * E + e] * w1[(long)d * E + e];
        dX[((long)h * B + b) * D + d] = acc;
      }
    for (int d = 0; d < D; ++d)
      for (int e = 0; e < E; ++e) {
        double acc = 0.0;
        for (int b = 0; b < B; ++b) acc += x[(long)b * D + d] * dZ[(long)b * E + e];
        dW1[((long)h * D + d) * E + e] = acc;
      }
    for (int e = 0; e < E; ++e)
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int b = 0; b < B; ++b) acc += act_f(Z[(long)b * E + e], act) * go[(long)b * D + d];
        dW2[((long)h * E + e) * D + d] = acc;
      }
  }
  free(Z);
  free(dZ);
}
