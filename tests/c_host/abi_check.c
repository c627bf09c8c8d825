/* Plain C99 host of the C ABI: includes include/flashspec_hip.h, links libflashspec_hip.so and
 * makes the calls that need no GPU (queries, and arguments rejected before any launch).
 * Prints one line per check; exit status 0 when all hold. */
#include <stdio.h>
#include <string.h>

#include "flashspec_hip.h"

static int failures = 0;

static void check(int ok, const char* what) {
  printf("%s %s\n", ok ? "ok" : "FAIL", what);
  if (!ok) ++failures;
}

int main(void) {
  check(fs_abi_version() == 2, "fs_abi_version() == 2");
  check(fs_decode_workspace_bytes(256, 16, 128) == (int64_t)256 * 16 * 130 * 4, "workspace bytes");
  check(fs_decode_tiled_path(128, 16, 16) == 1 && fs_decode_tiled_path(34, 16, 16) == 0, "tiled path query");
  check(fs_tree_mfma_path(128, 16, 16) == 1 && fs_tree_mfma_path(96, 16, 16) == 0, "tree path query");
  /* head_dim 0: rejected before launch, with a message */
  int rc = fs_paged_decode_i8((const void*)1, FS_F16, (const int8_t*)1, (const float*)1, (const int16_t*)1,
                              (const int8_t*)1, (const float*)1, (const int16_t*)1, (const void*)1, 8, 4,
                              (const int64_t*)1, (void*)1, NULL, 0, 1, 1, 0, 4, 16, 16, 64, 0.1f, 4, 1, 4, NULL);
  check(rc == FS_ERR_INVALID && strstr(fs_last_error(), "head_dim") != NULL, "invalid head_dim rejected");
  /* unsupported q dtype code in quantize */
  rc = fs_quantize_i8((const void*)1, 9, 1, 16, 128, 16, (int8_t*)1, (float*)1, (int16_t*)1, NULL);
  check(rc == FS_ERR_INVALID && fs_last_error()[0] != '\0', "invalid dtype rejected");
  return failures == 0 ? 0 : 1;
}
