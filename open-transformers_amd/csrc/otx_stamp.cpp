// Build provenance of libotx_attn.so, stamped at build time.
//
// The analogue of repop.build_info() (src/pretrain/cli/audit_replay.py:1508-1511
// of the reference records it with every replay): the commit of the source
// tree the library was built from, whether that tree differed from the
// commit, and a digest of the compiled sources and flags.  The build script
// passes the three values as macros; a build outside a git checkout stamps
// "unknown".  Host-only translation unit (no device code), compiled by the
// host compiler and linked into the library.
#ifndef OTX_STAMP_COMMIT
#define OTX_STAMP_COMMIT "unknown"
#endif
#ifndef OTX_STAMP_DIRTY
#define OTX_STAMP_DIRTY "null"
#endif
#ifndef OTX_STAMP_SOURCES
#define OTX_STAMP_SOURCES "unknown"
#endif

extern "C" const char* otx_build_info(void) {
  static const char info[] =
      "{\"library\": \"otx_attn\", \"backends\": [\"rocm\"], \"device_type\": \"cuda\", \"arch\": \"gfx950\", "
      "\"contract\": \"otx-attn-v1\", \"dtypes\": [\"float32\", \"bfloat16\"], \"head_dims\": [64, 128], "
      "\"block\": 32, \"atomics\": false, \"commit\": \"" OTX_STAMP_COMMIT "\", \"dirty\": " OTX_STAMP_DIRTY
      ", \"sources_blake2b\": \"" OTX_STAMP_SOURCES "\"}";
  return info;
}
