/* A plain C caller of the library: what a C / C++ host (or a cgo / JNI / N-API
 * stub) binds.  Host-only calls, so it runs without a GPU: the ABI version, the
 * workspace query of the fast GEMV, and an invalid call that must fail closed
 * with FX_EINVAL and a message.  Exit status 0 when every check holds. */
#include <stdio.h>
#include <string.h>

#include "fluxbin_amd.h"

int main(void) {
  int failures = 0;
  const int version = fx_abi_version();
  printf("abi %d\n", version);
  /* the workspace covering both arithmetics at q_proj's shape (the structural
     MFMA route needs none there; the decoded_bf16 table route its split partials) */
  const size_t ws = fx_w3_gemv_workspace_bytes(1, 4096, 4096);
  printf("workspace %zu\n", ws);
  if (ws % 256 != 0) ++failures;
  /* null payload: rejected on the host before any device call */
  const int rc = fx_w3_gemv(NULL, FX_BF16, NULL, NULL, FX_F16, NULL, NULL, NULL, 0, NULL, 1, 4096, 4096,
                            FX_ARITH_STRUCTURAL, NULL);
  const char* message = fx_last_error();
  printf("rc %d: %s\n", rc, message);
  if (rc != FX_EINVAL || strstr(message, "non-null") == NULL) ++failures;
  /* K not a multiple of 128 */
  static unsigned char dummy[64] __attribute__((aligned(16)));
  const int rc2 = fx_w3_gemv(dummy, FX_BF16, dummy, dummy, FX_F16, NULL, NULL, NULL, 0, dummy, 1, 64, 200,
                             FX_ARITH_STRUCTURAL, NULL);
  printf("rc %d: %s\n", rc2, fx_last_error());
  if (rc2 != FX_EINVAL || strstr(fx_last_error(), "multiple of 128") == NULL) ++failures;
  return failures;
}
