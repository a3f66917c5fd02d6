/* The C integration of libphantom_attn.so with no torch and no C++: includes both public headers
 * as C99, links against the library and makes calls that need no GPU (the version string, argument
 * validation of every fused entry's error path, the kernel description and the tile library's
 * count). Built and run by tests/test_api.py::test_c_abi_example_builds_and_runs. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "phantom_attn.h"
#include "phantom_attn_tiles.h"

static int fails = 0;

static void expect(int cond, const char* what) {
  if (!cond) {
    fprintf(stderr, "FAILED: %s (last error: %s)\n", what, pa_last_error());
    ++fails;
  }
}

int main(void) {
  const char* v = pa_version();
  expect(v != NULL && strstr(v, "gfx950") != NULL, "pa_version names gfx950");
  /* null tensors: rejected before any HIP call */
  int rc = pa_fused_tc_fwd(NULL, NULL, NULL, NULL, PA_DTYPE_BF16, PA_DTYPE_F32, 1, 64, 128, 0, NULL);
  expect(rc == PA_ERR_INVALID && strstr(pa_last_error(), "null") != NULL, "null pointers -> PA_ERR_INVALID");
  /* an aligned stand-in pointer that is never dereferenced: the head dimension fails first */
  void* p = (void*)(uintptr_t)256;
  rc = pa_fused_tc_fwd(p, p, p, p, PA_DTYPE_F16, PA_DTYPE_F16, 1, 64, 96, 0, NULL);
  expect(rc == PA_ERR_UNSUPPORTED && strstr(pa_last_error(), "head dimension") != NULL, "d = 96 -> PA_ERR_UNSUPPORTED");
  rc = pa_fused_fwd(p, p, p, p, PA_DTYPE_F32, PA_DTYPE_F32, 0, 64, 64, 0, NULL);
  expect(rc == PA_ERR_INVALID, "empty batch -> PA_ERR_INVALID");
  const char* desc = pa_fused_tc_kernel(PA_DTYPE_BF16, PA_DTYPE_BF16, 128, 4096, 128, 0);
  expect(desc != NULL && strncmp(desc, "fa_mfma_fwd<bf16, D=128, BM=256", 31) == 0, "pa_fused_tc_kernel describes C4");
  expect(pa_tiles_count() > 0, "the tile library lists its candidates");
  if (fails == 0) printf("c abi ok: %s\n", v);
  return fails == 0 ? 0 : 1;
}
