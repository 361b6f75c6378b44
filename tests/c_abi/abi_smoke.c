/* A non-Python caller of libparoquant_hip.so: plain C against
 * include/paroquant_hip.h.  It makes only host-side calls (version, the
 * workspace-size rules, argument checks that fail before any launch), so it
 * runs without a GPU.  tests/test_c_abi.py builds and runs it. */
#include <stdio.h>
#include <string.h>

#include "paroquant_hip.h"

static int fails = 0;
#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      printf("FAIL line %d: %s\n", __LINE__, #cond);                  \
      fails++;                                                        \
    }                                                                 \
  } while (0)

int main(void) {
  CHECK(pq_abi_version() == PQ_ABI_VERSION);
  /* decode sizes: rotated fp32 rows (256-byte aligned) + per-group maxima */
  CHECK(pq_w4a8_linear_workspace_size(1, 4096, 4096, 8) == 4096 * 4 + 32 * 4);
  /* row path: int8 codes + token scales */
  CHECK(pq_w4a8_linear_workspace_size(65, 4096, 4096, 8) == 65 * 4096 + 65 * 4);
  CHECK(pq_w4a8_linear_group_workspace_size(65, 4096, 3) == 3 * (65 * 4096 + 65 * 4));
  CHECK(pq_w4a16_linear_workspace_size(64, 4096) == 64 * 4096 * 2);
  CHECK(pq_w4a8_linear_split_path(1, 4096) == 1 && pq_w4a8_linear_split_path(16, 4096) == 1 &&
        pq_w4a8_linear_split_path(64, 4096) == 1 && pq_w4a8_linear_split_path(65, 4096) == 0);

  /* a bad group size is refused on the host, with a message */
  void* p = (void*)(size_t)256;
  int st = pq_w4a8_gemm(p, p, p, p, NULL, 0, p, PQ_BF16, 4, 64, 256, 64, NULL, 0, NULL);
  CHECK(st == PQ_ERR_UNSUPPORTED);
  CHECK(strstr(pq_last_error(), "group_size") != NULL);
  /* a linear without workspace is refused before anything is launched */
  st = pq_w4a8_linear(p, PQ_BF16, p, p, NULL, p, p, NULL, 0, p, PQ_BF16, 64, 4096, 4096, 8,
                      PQ_RQ_INPUT_FP16 | PQ_RQ_MATERIALIZE_FP16, NULL, 0, NULL);
  CHECK(st == PQ_ERR_WORKSPACE);
  /* a group through the member table: an unknown prologue mode */
  pq_linear_member m;
  memset(&m, 0, sizeof m);
  m.rot_idx = p; m.rot_cs = p; m.wpack = p; m.wmeta = p; m.y = p; m.n = 64;
  st = pq_w4a8_linear_group_fused(p, p, NULL, 0.0f, 9, NULL, NULL, PQ_BF16, &m, 1, 0, PQ_BF16, 1, 4096, 8, 0, p,
                                  1 << 20, NULL);
  CHECK(st == PQ_ERR_ARG);
  /* empty inputs are no-ops */
  CHECK(pq_rotate_mxfp4(p, p, p, p, p, NULL, 0, 256, 8, 128, PQ_BF16, NULL) == PQ_OK);
  CHECK(pq_w4a16_gemm(p, p, p, NULL, 0, p, PQ_F16, 0, 64, 256, 128, NULL) == PQ_OK);

  printf("%s (%d failures)\n", fails ? "FAILED" : "ok", fails);
  return fails ? 1 : 0;
}
