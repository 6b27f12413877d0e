/*
 * Plugin host harness: loads the extension libraries the way Triton loads a
 * pass plugin (dlopen of the path in TRITON_PASS_PLUGIN_PATH, README.md:114-121
 * of the reference) and drives them only through dlsym'd C-ABI entry points:
 *   tritonEnumeratePluginPasses (two-call protocol), tritonRegisterPluginPass,
 *   tritonAddPluginPass, then runs the pass manager over a dot plan.
 * Usage: plugin_host <lib dir>.  Prints one line per fact; exit 0 on success.
 */
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "triton_ext/TritonExtPassInfra.h"
#include "triton_ext/tx_dot.h"

#define SYM(h, T, name) T name = (T)dlsym(h, #name); if (!name) { printf("missing %s\n", #name); return 2; }

typedef TritonPluginResult (*enum_fn)(uint32_t *, const char **);
typedef TritonPluginResult (*add_fn)(TxPassManager *, const char *);
typedef TritonPluginResult (*reg_fn)(const char *);
typedef TxPassManager *(*pmc_fn)(void);
typedef void (*pmd_fn)(TxPassManager *);
typedef int (*pmr_fn)(TxPassManager *, tx_dot_plan *);
typedef uint32_t (*pms_fn)(const TxPassManager *);
typedef const char *(*pmn_fn)(const TxPassManager *, uint32_t);
typedef int (*pmp_fn)(TxPassManager *, const char *);

int main(int argc, char **argv) {
  if (argc < 2) return 2;
  char path[4096];
  snprintf(path, sizeof path, "%s/libTritonExtPassInfra.so", argv[1]);
  void *infra = dlopen(path, RTLD_NOW | RTLD_GLOBAL);
  if (!infra) { printf("dlopen infra: %s\n", dlerror()); return 2; }
  SYM(infra, enum_fn, tritonEnumeratePluginPasses);
  SYM(infra, add_fn, tritonAddPluginPass);
  SYM(infra, reg_fn, tritonRegisterPluginPass);
  SYM(infra, pmc_fn, txPassManagerCreate);
  SYM(infra, pmd_fn, txPassManagerDestroy);
  SYM(infra, pmr_fn, txPassManagerRun);
  SYM(infra, pms_fn, txPassManagerSize);
  SYM(infra, pmn_fn, txPassManagerPassName);
  SYM(infra, pmp_fn, txPassManagerParsePipeline);

  uint32_t n = 99;
  if (tritonEnumeratePluginPasses(&n, NULL) != TP_SUCCESS) return 3;
  printf("before_load count=%u\n", n);
  if (tritonEnumeratePluginPasses(NULL, NULL) != TP_GENERIC_FAILURE) return 3;
  printf("null_count failure ok\n");

  const char *plugins[] = {"libloop_split.so", "libarith_intensity.so"};
  for (int i = 0; i < 2; ++i) {
    snprintf(path, sizeof path, "%s/%s", argv[1], plugins[i]);
    if (!dlopen(path, RTLD_NOW | RTLD_GLOBAL)) { printf("dlopen %s: %s\n", plugins[i], dlerror()); return 2; }
  }
  if (tritonEnumeratePluginPasses(&n, NULL) != TP_SUCCESS) return 3;
  const char **names = calloc(n, sizeof(char *));
  if (tritonEnumeratePluginPasses(&n, names) != TP_SUCCESS) return 3;
  printf("after_load count=%u", n);
  for (uint32_t i = 0; i < n; ++i) printf(" %s", names[i]);
  printf("\n");

  if (tritonRegisterPluginPass("no_such_pass") != TP_GENERIC_FAILURE) return 4;
  if (tritonRegisterPluginPass("loop_split") != TP_SUCCESS) return 4;
  if (tritonRegisterPluginPass("arith_intensity") != TP_SUCCESS) return 4;
  printf("register ok\n");

  TxPassManager *pm = txPassManagerCreate();
  if (tritonAddPluginPass(pm, "no_such_pass") != TP_GENERIC_FAILURE) return 5;
  if (tritonAddPluginPass(NULL, "loop_split") != TP_GENERIC_FAILURE) return 5;
  if (tritonAddPluginPass(pm, "arith_intensity") != TP_SUCCESS) return 5;
  if (tritonAddPluginPass(pm, "loop_split") != TP_SUCCESS) return 5;
  printf("pm size=%u", txPassManagerSize(pm));
  for (uint32_t i = 0; i < txPassManagerSize(pm); ++i) printf(" %s", txPassManagerPassName(pm, i));
  printf("\n");

  tx_dot_plan plan;
  memset(&plan, 0, sizeof plan);
  plan.desc.M = 4096; plan.desc.N = 4096; plan.desc.K = 4000;
  plan.desc.a_type = plan.desc.b_type = TX_BF16; plan.desc.c_type = TX_BF16;
  if (txPassManagerRun(pm, &plan) != 0) return 6;
  printf("plan block=%dx%dx%d k_split=%lld main=%d tail=%d bound=%d passes=%d\n",
         plan.desc.block_m, plan.desc.block_n, plan.desc.block_k, (long long)plan.k_split,
         plan.k_main_steps, plan.k_tail, plan.bound, plan.passes_run);
  txPassManagerDestroy(pm);

  /* textual pipeline, available after registration */
  pm = txPassManagerCreate();
  if (txPassManagerParsePipeline(pm, "tx-arith-intensity, -triton-loop-split") != 0) return 7;
  if (txPassManagerParsePipeline(pm, "triton-loop-split,bogus") == 0) return 7;
  printf("pipeline size=%u %s %s\n", txPassManagerSize(pm), txPassManagerPassName(pm, 0),
         txPassManagerPassName(pm, 1));
  txPassManagerDestroy(pm);
  free(names);
  printf("OK\n");
  return 0;
}
