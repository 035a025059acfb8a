/* libtinyinfer_diag.so — machine-limit probes used by bench.py; no counterpart
 * in the reference and not part of the drop-in boundary.
 *
 * tia_diag_empty: enqueue one empty kernel on `stream` (launch-floor probe).
 * tia_diag_stream: enqueue a pure streaming read of wgs * per_wg bytes from
 *   `src` (16-byte aligned device memory), workgroup w reading bytes
 *   [w * per_wg, (w + 1) * per_wg) with `threads` threads (multiple of 64, at
 *   most 1024); `out` receives wgs * threads dwords.  per_wg must be a positive
 *   multiple of 1024.  Both return 0, or 1 on invalid arguments / launch error. */
#ifndef TINYINFER_AMD_DIAG_H
#define TINYINFER_AMD_DIAG_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
int tia_diag_empty(uintptr_t stream);
int tia_diag_stream(const void* src, unsigned* out, int64_t per_wg, int wgs, int threads, uintptr_t stream);
#ifdef __cplusplus
}
#endif
#endif
