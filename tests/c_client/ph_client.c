/*
 * A plain C client of libpalladium_hip.so: what a non-Python caller (a cgo
 * or JNI binding, a C++ XLA handler) sees. Built by tests/test_c_client.py
 * with gcc against include/palladium_hip.h only.
 *
 *   ph_client compile   compile a saxpy kernel for gfx950 (no GPU needed)
 *   ph_client dispatch  run it through ph_dispatch on host buffers,
 *                       through ph_dispatch_device on device buffers and
 *                       through ph_dispatch_noalloc (twice, the second
 *                       call smaller, then once too large to fit)
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "palladium_hip.h"

static const char *kSource =
    "extern \"C\" __global__ void __launch_bounds__(256)\n"
    "saxpy(const float* __restrict__ x, const float* __restrict__ y, float* __restrict__ o)\n"
    "{\n"
    "    const unsigned int i = blockIdx.x * 256u + threadIdx.x;\n"
    "    if (i >= 1000u) return;\n"
    "    o[i] = 2.5f * x[i] + y[i];\n"
    "}\n";

static int fail(const char *what, int rc, char *err) {
  fprintf(stderr, "%s failed (%d): %s\n", what, rc, err ? err : "");
  ph_free_error(err);
  return 1;
}

static int check(const float *x, const float *y, const float *o, int n) {
  for (int i = 0; i < n; ++i) {
    float want = 2.5f * x[i] + y[i];
    if (o[i] != want) {
      fprintf(stderr, "o[%d] = %g, want %g\n", i, o[i], want);
      return 1;
    }
  }
  return 0;
}

int main(int argc, char **argv) {
  const char *mode = argc > 1 ? argv[1] : "compile";
  char *err = NULL;
  printf("palladium_hip %s\n", ph_version());
  if (strcmp(mode, "compile") == 0) {
    void *code = NULL;
    size_t size = 0;
    int rc = ph_compile_code_object(kSource, strlen(kSource), "saxpy", PH_MATH_SAFE, NULL, &code, &size, &err);
    if (rc != PH_OK) return fail("ph_compile_code_object", rc, err);
    printf("compiled %zu bytes, ELF=%d\n", size, size > 4 && memcmp(code, "\x7f" "ELF", 4) == 0);
    ph_free_code_object(code);
    rc = ph_compile_code_object("not hip", 7, "k", 9, NULL, &code, &size, &err);
    printf("bad math mode -> %d (%s)\n", rc, err ? err : "");
    ph_free_error(err);
    return 0;
  }

  enum { N = 1000 };
  float *x = malloc(N * sizeof(float)), *y = malloc(N * sizeof(float)), *o = malloc(N * sizeof(float));
  for (int i = 0; i < N; ++i) {
    x[i] = (float)i * 0.25f;
    y[i] = 1.0f - (float)i;
  }
  const void *ins[2] = {x, y};
  size_t in_bytes[2] = {N * sizeof(float), N * sizeof(float)};
  void *outs[1] = {o};
  size_t out_bytes[1] = {N * sizeof(float)};
  /* One lane per element: grid = (1000,), 256-lane workgroups. */
  int rc = ph_dispatch(kSource, strlen(kSource), "saxpy", N, 1, 1, 256, 1, PH_MATH_SAFE, ins, in_bytes, 2, outs,
                       out_bytes, 1, &err);
  if (rc != PH_OK) return fail("ph_dispatch", rc, err);
  if (check(x, y, o, N)) return 1;
  printf("ph_dispatch ok\n");

  void *dx = NULL, *dy = NULL, *dout = NULL, *stream = NULL;
  if ((rc = ph_malloc(N * sizeof(float), &dx, &err)) || (rc = ph_malloc(N * sizeof(float), &dy, &err)) ||
      (rc = ph_malloc(N * sizeof(float), &dout, &err)) || (rc = ph_stream_create(&stream, &err)))
    return fail("allocation", rc, err);
  if ((rc = ph_memcpy_h2d(dx, x, N * sizeof(float), stream, &err)) ||
      (rc = ph_memcpy_h2d(dy, y, N * sizeof(float), stream, &err)))
    return fail("ph_memcpy_h2d", rc, err);
  const void *dins[2] = {dx, dy};
  void *douts[1] = {dout};
  memset(o, 0, N * sizeof(float));
  rc = ph_dispatch_device(kSource, strlen(kSource), "saxpy", N, 1, 1, 256, 1, PH_MATH_FAST, stream, dins, 2, douts, 1,
                          &err);
  if (rc != PH_OK) return fail("ph_dispatch_device", rc, err);
  if ((rc = ph_memcpy_d2h_wait(o, dout, N * sizeof(float), stream, &err))) return fail("ph_memcpy_d2h_wait", rc, err);
  /* FAST may fuse 2.5*x + y into one FMA: compare to within a rounding. */
  for (int i = 0; i < N; ++i) {
    float want = 2.5f * x[i] + y[i];
    float tol = 1e-6f * (2.5f * (x[i] < 0 ? -x[i] : x[i]) + (y[i] < 0 ? -y[i] : y[i])) + 1e-30f;
    float d = o[i] - want;
    if (d > tol || d < -tol) {
      fprintf(stderr, "device o[%d] = %g, want %g\n", i, o[i], want);
      return 1;
    }
  }
  printf("ph_dispatch_device ok\n");

  /* The allocation-free entry point: the kernel from the cache, operands
   * staged in the library's fixed per-GPU array. The kernel guards i < 1000,
   * so a shorter call gets a shorter grid and shorter buffers. */
  ph_kernel *k = NULL;
  if ((rc = ph_get_kernel(kSource, strlen(kSource), "saxpy", PH_MATH_SAFE, &k, &err))) return fail("ph_get_kernel", rc, err);
  for (int pass = 0; pass < 2; ++pass) {
    const int n = pass == 0 ? N : 300;
    size_t nb[2] = {n * sizeof(float), n * sizeof(float)}, ob[1] = {n * sizeof(float)};
    memset(o, 0, N * sizeof(float));
    rc = ph_dispatch_noalloc(k, n, 1, 1, 256, 1, NULL, ins, nb, 2, outs, ob, 1, &err);
    if (rc != PH_OK) return fail("ph_dispatch_noalloc", rc, err);
    if (check(x, y, o, n)) return 1;
    for (int i = n; i < N; ++i)
      if (o[i] != 0.0f) {
        fprintf(stderr, "o[%d] written past the output\n", i);
        return 1;
      }
  }
  size_t huge[2] = {ph_noalloc_scratch_bytes(), N * sizeof(float)};
  rc = ph_dispatch_noalloc(k, N, 1, 1, 256, 1, NULL, ins, huge, 2, outs, out_bytes, 1, &err);
  printf("oversized -> %d (%s)\n", rc, err ? err : "");
  ph_free_error(err);
  err = NULL;
  if (rc == PH_OK) return 1;
  printf("ph_dispatch_noalloc ok\n");
  ph_free(dx);
  ph_free(dy);
  ph_free(dout);
  ph_stream_destroy(stream);
  free(x);
  free(y);
  free(o);
  return 0;
}
