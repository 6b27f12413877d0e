/*
 * triton-ext plugin surface, MI355X build.
 *
 * The four entry points below keep the names, argument meaning, return codes
 * and two-call enumeration protocol of the reference's pass registry:
 *   tritonAddPluginPass         R:infra/pass/TritonExtPassInfra.h:11-12
 *                               (impl R:infra/pass/TritonExtPassInfra.cpp:19-26)
 *   tritonRegisterPluginPass    R:infra/pass/TritonExtPassInfra.h:14-15
 *                               (impl R:infra/pass/TritonExtPassInfra.cpp:28-35)
 *   tritonEnumeratePluginPasses R:infra/pass/TritonExtPassInfra.h:17-18
 *                               (impl R:infra/pass/TritonExtPassInfra.cpp:37-52)
 *   TritonExtLoadPass           R:infra/pass/TritonExtPassInfra.h:24-26
 *                               (impl R:infra/pass/TritonExtPassInfra.cpp:7-14)
 * ("R:" = the triton-ext source tree.)
 *
 * Differences that are deliberate:
 *  - MLIR is not part of this build, so `mlir::PassManager *` becomes the
 *    opaque `TxPassManager *` declared here.  Extensions append their pass to
 *    it with txPassManagerAddPass(); the pass runs over a tx_dot_plan (the
 *    planning record of one tiled dot, include/triton_ext/tx_dot.h).
 *  - `TritonPluginResult` / `TRITON_PLUGIN_API` come from Triton's
 *    PluginUtils.h, which the reference includes but does not ship
 *    (R:infra/pass/TritonExtPassInfra.h:8).  They are defined here with
 *    TP_SUCCESS = 0 and TP_GENERIC_FAILURE = 1.
 *  - tritonEnumeratePluginPasses fills every slot (the reference writes every
 *    name to passNames[0], R:infra/pass/TritonExtPassInfra.cpp:47-50), and a
 *    duplicate TritonExtLoadPass replaces the earlier entry instead of
 *    growing the name table past the maps' size.
 *  - The registry is guarded by a mutex, so registration from concurrent
 *    dlopen() calls is safe.
 */
#ifndef TRITON_EXT_AMD_PASS_INFRA_H
#define TRITON_EXT_AMD_PASS_INFRA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum TritonPluginResult {
  TP_SUCCESS = 0,
  TP_GENERIC_FAILURE = 1,
} TritonPluginResult;

#define TRITON_PLUGIN_API                                                      \
  __attribute__((visibility("default"))) TritonPluginResult

/* Opaque pass manager (stands where mlir::PassManager stands in the
 * reference). */
typedef struct TxPassManager TxPassManager;
/* The IR a pass runs on: the plan of one tiled dot. */
typedef struct tx_dot_plan tx_dot_plan;
/* A pass body: returns 0 on success, non-zero to stop the pipeline. */
typedef int (*TxPassRunFunc)(tx_dot_plan *plan);

/* ---- Triton-side API (R:infra/pass/TritonExtPassInfra.h:10-18) ---------- */

/* Add the extension pass registered under `passName` to `pm`.
 * TP_GENERIC_FAILURE if no extension of that name is loaded or `pm` is NULL. */
TRITON_PLUGIN_API
tritonAddPluginPass(TxPassManager *pm, const char *passName);

/* Run the extension's registration hook, which makes its pass argument
 * (e.g. "triton-loop-split") available to txPassManagerParsePipeline().
 * TP_GENERIC_FAILURE for an unknown name. */
TRITON_PLUGIN_API
tritonRegisterPluginPass(const char *passName);

/* Two-call protocol: with passNames == NULL only *passCount is written; then
 * the caller passes an array of *passCount entries, filled in load order.
 * TP_GENERIC_FAILURE if passCount is NULL.  Names are borrowed and stay
 * valid while the extension library stays loaded. */
TRITON_PLUGIN_API
tritonEnumeratePluginPasses(uint32_t *passCount, const char **passNames);

/* ---- Extension-side API (R:infra/pass/TritonExtPassInfra.h:20-26) ------- */

typedef void (*TritonExtRegisterPassFunc)(void);
typedef void (*TritonExtAddPassFunc)(TxPassManager *);

/* Called from an extension's static initialiser while it is dlopen()ed.
 * Always succeeds for non-NULL arguments; a second load of the same name
 * replaces the first. */
TRITON_PLUGIN_API
TritonExtLoadPass(const char *passName, TritonExtRegisterPassFunc registerFunc,
                  TritonExtAddPassFunc addFunc);

/* ---- Pass manager (no counterpart in the reference: MLIR supplies it) --- */

__attribute__((visibility("default"))) TxPassManager *txPassManagerCreate(void);
__attribute__((visibility("default"))) void txPassManagerDestroy(TxPassManager *pm);
/* Append a pass.  `argName` is the pass argument (e.g. "triton-loop-split"). */
__attribute__((visibility("default"))) int
txPassManagerAddPass(TxPassManager *pm, const char *argName, TxPassRunFunc run);
/* Number of passes and the argument name of pass `i` (NULL if out of range). */
__attribute__((visibility("default"))) uint32_t txPassManagerSize(const TxPassManager *pm);
__attribute__((visibility("default"))) const char *
txPassManagerPassName(const TxPassManager *pm, uint32_t i);
/* Run the passes in order; stops at and returns the first non-zero status. */
__attribute__((visibility("default"))) int txPassManagerRun(TxPassManager *pm,
                                                            tx_dot_plan *plan);

/* Textual pipelines ("triton-loop-split,tx-arith-intensity"), the role
 * mlir::registerPass plays for the reference (R:infra/pass/TritonExtPass.cpp:31-35).
 * Registration hooks call txRegisterPassArgument; txPassManagerParsePipeline
 * appends the named passes.  Returns 0, or 1 if an argument is unknown
 * (nothing is appended then). */
__attribute__((visibility("default"))) int
txRegisterPassArgument(const char *argName, TxPassRunFunc run);
__attribute__((visibility("default"))) int
txPassManagerParsePipeline(TxPassManager *pm, const char *pipeline);

/* triton-ext.conf: `name;status[;hash]` (R:cmake/utils.cmake:92-136).
 * Reads `<dir>/triton-ext.conf`, falling back to `<dir>/triton_ext.conf`
 * (both spellings appear in the reference's docs).  Returns 0 on success,
 * 1 if neither file exists or the name field is empty. */
__attribute__((visibility("default"))) int
txReadExtConf(const char *dir, char *name, uint32_t nameCap, char *status,
              uint32_t statusCap, char *hash, uint32_t hashCap);

#ifdef __cplusplus
}
#endif

#endif /* TRITON_EXT_AMD_PASS_INFRA_H */
