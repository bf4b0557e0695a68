/*
 * pjrt_mi355x.h — the drop-in boundary of the MI355X PJRT plugin.
 *
 * libpjrt_mi355x.so exports exactly one symbol, like the reference plugin
 * (Lazarus-931/mccl-jax src/pjrt/api/pjrt_c_api.h:6 and the visibility rules
 * of its CMakeLists.txt:8-10):
 *
 *   const PJRT_Api* GetPjrtApi(void);
 *
 * It returns a process-lifetime table of the PJRT C API, version 0.55 (the
 * version the reference pins: third_party/xla/pjrt/c/PROVENANCE.md:6-8),
 * with all 100 function slots non-null.  jaxlib loads it through
 *   jax._src.xla_bridge.register_plugin("mi355x", library_path=".../libpjrt_mi355x.so")
 * exactly as the reference is loaded (README.md:25-32).  The struct layouts
 * are those of the PJRT C API header; this repository declares them in
 * mccl-jax_amd/src/pjrt/api/pjrt_abi.h.
 */
#ifndef MI355X_PJRT_MI355X_H_
#define MI355X_PJRT_MI355X_H_

#ifdef __cplusplus
extern "C" {
#endif

typedef struct PJRT_Api PJRT_Api;

/* Replaces: src/pjrt/api/pjrt_c_api.h:6 / pjrt_c_api.cc:877-989 (GetPjrtApi). */
const PJRT_Api* GetPjrtApi(void);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_PJRT_MI355X_H_ */
