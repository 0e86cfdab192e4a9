// Option handling of the C ABI: defaults, name=value parsing and validation.
//
// Option names, defaults and ranges follow the reference pipeline and pass
// options (include/sparsewave/Target/AMDGPU/Pipelines.h:108-191,
// include/sparsewave/Dialect/SparseWave/Transforms/Passes.td:146-241).  The
// validation order and the wording of the diagnostics follow
// ConvertSparseWaveToGPU::runOnOperation
// (lib/Dialect/SparseWave/Transforms/SparseWaveToGPU.cpp:1265-1397) and
// ScheduleSparseWavePosition::runOnOperation
// (lib/Dialect/SparseWave/Transforms/SparsePositionScheduling.cpp:411-465).
// The reference requires Wave32 for every cooperative mapping because it
// targets gfx1101; gfx950 executes Wave64 only, so the same checks require 64.
#include "sw_internal.h"

#include <cctype>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

namespace {
thread_local std::string g_last_error;

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int set_string(char *dst, size_t cap, const char *value) {
  size_t n = std::strlen(value);
  if (n + 1 > cap)
    return sw::fail(SW_ERR_INVALID_OPTION, "option value '%s' is too long",
                    value);
  std::memcpy(dst, value, n + 1);
  return SW_OK;
}

int parse_int(const char *name, const char *value, int64_t *out) {
  errno = 0;
  char *end = nullptr;
  long long v = std::strtoll(value, &end, 10);
  if (errno != 0 || end == value || *end != '\0')
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "option '%s' expects an integer, but got '%s'", name,
                    value);
  *out = (int64_t)v;
  return SW_OK;
}

int check_block(const char *what, int64_t v) {
  if (v < 1 || v > 1024)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "%s block size must be between 1 and 1024, but got %lld",
                    what, (long long)v);
  return SW_OK;
}
} // namespace

namespace sw {

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

} // namespace sw

extern "C" {

void sw_options_init(sw_options *o) {
  std::memset(o, 0, sizeof(*o));
  std::strcpy(o->spmv_mapping, "thread-per-row");
  o->spmv_block_size = 256;
  o->spmv_position_chunk_size = 1;
  std::strcpy(o->spmv_position_reduction, "atomic");
  o->position_block_size = 256;
  std::strcpy(o->spmm_mapping, "thread-per-output");
  o->spmm_block_size = 256;
  o->spmm_tile_size = 4;
  o->spmm_position_chunk_size = 1;
  o->sddmm_block_size = 256;
  o->row_reduction_block_size = 256;
  o->rowwise_map_block_size = 256;
  o->elementwise_block_size = 256;
  o->wavefront_size = 64;
  o->spmv_lanes_per_row = 64;
  o->spmv_positions_per_lane = 1;
  o->spmm_lanes_per_row = 64;
  o->bsr_use_mfma = 1;
  o->sddmm_lanes_per_row = 1;
  o->spmm_positions_per_lane = 4;
  std::strcpy(o->sddmm_mapping, "thread-per-row");
}

int sw_options_set(sw_options *o, const char *name, const char *value) {
  if (!o || !name || !value)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null option argument");
  std::string n(name);
  struct IntOpt {
    const char *pass_name;
    const char *pipeline_name;
    int64_t *field;
  } ints[] = {
      {"block-size", "spmv-block-size", &o->spmv_block_size},
      {nullptr, "spmv-position-chunk-size", &o->spmv_position_chunk_size},
      {"thread-chunk-size", nullptr, &o->spmv_position_chunk_size},
      {"position-block-size", "position-block-size", &o->position_block_size},
      {"spmm-block-size", "spmm-block-size", &o->spmm_block_size},
      {"spmm-tile-size", "spmm-tile-size", &o->spmm_tile_size},
      {nullptr, "spmm-position-chunk-size", &o->spmm_position_chunk_size},
      {"sddmm-block-size", "sddmm-block-size", &o->sddmm_block_size},
      {"row-reduction-block-size", "row-reduction-block-size",
       &o->row_reduction_block_size},
      {"rowwise-map-block-size", "rowwise-map-block-size",
       &o->rowwise_map_block_size},
      {"elementwise-block-size", "elementwise-block-size",
       &o->elementwise_block_size},
      {"wave-size", "wavefront-size", &o->wavefront_size},
      {"spmv-lanes-per-row", "spmv-lanes-per-row", &o->spmv_lanes_per_row},
      {"spmv-positions-per-lane", "spmv-positions-per-lane",
       &o->spmv_positions_per_lane},
      {"spmm-lanes-per-row", "spmm-lanes-per-row", &o->spmm_lanes_per_row},
      {"bsr-use-mfma", "bsr-use-mfma", &o->bsr_use_mfma},
      {"sddmm-lanes-per-row", "sddmm-lanes-per-row", &o->sddmm_lanes_per_row},
      {"spmm-positions-per-lane", "spmm-positions-per-lane",
       &o->spmm_positions_per_lane},
  };
  for (const IntOpt &opt : ints) {
    if ((opt.pass_name && n == opt.pass_name) ||
        (opt.pipeline_name && n == opt.pipeline_name))
      return parse_int(name, value, opt.field);
  }
  if (n == "spmv-mapping" || n == "mapping")
    return set_string(o->spmv_mapping, sizeof(o->spmv_mapping), value);
  if (n == "spmv-position-reduction" || n == "thread-reduction")
    return set_string(o->spmv_position_reduction,
                      sizeof(o->spmv_position_reduction), value);
  if (n == "spmm-mapping")
    return set_string(o->spmm_mapping, sizeof(o->spmm_mapping), value);
  if (n == "sddmm-mapping")
    return set_string(o->sddmm_mapping, sizeof(o->sddmm_mapping), value);
  if (n == "chip") {
    if (std::strcmp(value, "gfx950") != 0)
      return sw::fail(SW_ERR_INVALID_OPTION,
                      "this library is built for gfx950, but chip=%s", value);
    return SW_OK;
  }
  // Target and backend options of the reference pipeline that have no
  // meaning for a prebuilt HIP library (Pipelines.h:27-99, 179-190).
  static const char *ignored[] = {"rocm-path",
                                  "triple",
                                  "features",
                                  "opt-level",
                                  "abi",
                                  "binary-format",
                                  "kernel-bare-ptr-calling-convention",
                                  "lower-host",
                                  "sink-launch-index-computations",
                                  "prepare-gpu-bare-ptr-abi",
                                  "index-bitwidth",
                                  "use-bare-ptr-memref-call-conv"};
  for (const char *ig : ignored)
    if (n == ig)
      return SW_OK;
  return sw::fail(SW_ERR_INVALID_OPTION, "unknown option '%s'", name);
}

int sw_options_parse(sw_options *o, const char *text) {
  if (!o || !text)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null option argument");
  std::string s(text);
  size_t lb = s.find('{');
  if (lb != std::string::npos) {
    size_t rb = s.rfind('}');
    if (rb == std::string::npos || rb < lb)
      return sw::fail(SW_ERR_INVALID_OPTION, "unbalanced braces in '%s'",
                      text);
    s = s.substr(lb + 1, rb - lb - 1);
  }
  size_t i = 0;
  while (i < s.size()) {
    while (i < s.size() && std::isspace((unsigned char)s[i]))
      ++i;
    if (i >= s.size())
      break;
    size_t j = i;
    while (j < s.size() && !std::isspace((unsigned char)s[j]))
      ++j;
    std::string tok = s.substr(i, j - i);
    size_t eq = tok.find('=');
    if (eq == std::string::npos)
      return sw::fail(SW_ERR_INVALID_OPTION,
                      "expected name=value, but got '%s'", tok.c_str());
    std::string name = tok.substr(0, eq), value = tok.substr(eq + 1);
    int rc = sw_options_set(o, name.c_str(), value.c_str());
    if (rc != SW_OK)
      return rc;
    i = j;
  }
  return SW_OK;
}

int sw_validate_options(const sw_options *o) {
  if (!o)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null options");
  std::string spmv(o->spmv_mapping), spmm(o->spmm_mapping),
      reduction(o->spmv_position_reduction);
  bool spmv_row = spmv == "thread-per-row" || spmv == "wave-per-row" ||
                  spmv == "block-per-row";
  bool spmv_pos = spmv == "thread-per-position" || spmv == "wave-per-position";
  // Wave64 extension: rows owned by the wave whose nonzero chunk holds
  // their first position
  bool spmv_owner = spmv == "wave-per-row-balanced";
  if (!spmv_row && !spmv_pos && !spmv_owner)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "unsupported SpMV mapping strategy '%s'; expected "
                    "'thread-per-row', 'wave-per-row', 'block-per-row', "
                    "'thread-per-position', 'wave-per-position', or "
                    "'wave-per-row-balanced'",
                    o->spmv_mapping);
  if (spmm != "thread-per-output" && spmm != "wave-per-row-tile" &&
      spmm != "thread-per-position" && spmm != "wave-per-position" &&
      spmm != "row-tile-mfma" && spmm != "wave-per-row-balanced" &&
      spmm != "wave-per-row-tile-lds")
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "unsupported SpMM mapping strategy '%s'; expected "
                    "'thread-per-output', 'wave-per-row-tile', "
                    "'thread-per-position', 'wave-per-position', "
                    "'row-tile-mfma', 'wave-per-row-balanced', or "
                    "'wave-per-row-tile-lds'",
                    o->spmm_mapping);
  std::string sddmm(o->sddmm_mapping);
  if (sddmm != "thread-per-row" && sddmm != "wave-per-row" &&
      sddmm != "row-tile-mfma")
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "unsupported SDDMM mapping strategy '%s'; expected "
                    "'thread-per-row', 'wave-per-row', or 'row-tile-mfma'",
                    o->sddmm_mapping);
  int rc;
  if ((rc = check_block("SpMV", o->spmv_block_size)))
    return rc;
  if ((rc = check_block("position-parallel", o->position_block_size)))
    return rc;
  if ((rc = check_block("SpMM", o->spmm_block_size)))
    return rc;
  if (o->spmm_tile_size < 1 || o->spmm_tile_size > 32)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "SpMM tile size must be between 1 and 32, but got %lld",
                    (long long)o->spmm_tile_size);
  if ((rc = check_block("SDDMM", o->sddmm_block_size)))
    return rc;
  if ((rc = check_block("CSR row-reduction", o->row_reduction_block_size)))
    return rc;
  if ((rc = check_block("CSR row-wise map", o->rowwise_map_block_size)))
    return rc;
  if ((rc = check_block("elementwise", o->elementwise_block_size)))
    return rc;
  const int64_t w = o->wavefront_size;
  bool wave_spmm = spmm == "wave-per-row-tile" ||
                   spmm == "wave-per-position" || spmm == "row-tile-mfma" ||
                   spmm == "wave-per-row-balanced" ||
                   spmm == "wave-per-row-tile-lds";
  bool wave_spmv = spmv == "wave-per-row" || spmv == "block-per-row" ||
                   spmv == "wave-per-position" || spmv_owner;
  if ((wave_spmm || wave_spmv) && w != 64)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "%s currently requires Wave64 on gfx950, but got wave "
                    "size %lld",
                    wave_spmm ? o->spmm_mapping : o->spmv_mapping,
                    (long long)w);
  if (w != 64)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "gfx950 executes Wave64 only, but got wave size %lld",
                    (long long)w);
  if (wave_spmm && o->spmm_block_size % w != 0)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "%s requires the SpMM block size to be a multiple of "
                    "%lld, but got %lld",
                    o->spmm_mapping, (long long)w,
                    (long long)o->spmm_block_size);
  if (wave_spmv && o->spmv_block_size % w != 0) {
    if (spmv == "wave-per-position")
      return sw::fail(SW_ERR_INVALID_OPTION,
                      "wave position mapping requires the block size to be a "
                      "multiple of %lld, but got %lld",
                      (long long)w, (long long)o->spmv_block_size);
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "%s requires the SpMV block size to be a multiple of "
                    "%lld, but got %lld",
                    o->spmv_mapping, (long long)w,
                    (long long)o->spmv_block_size);
  }
  if (o->spmv_position_chunk_size < 1)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "thread position chunk size must be positive, but got "
                    "%lld",
                    (long long)o->spmv_position_chunk_size);
  if (reduction != "atomic" && reduction != "segmented")
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "unsupported thread position reduction '%s'; expected "
                    "'atomic' or 'segmented'",
                    o->spmv_position_reduction);
  if (spmv == "wave-per-position" && o->spmv_position_chunk_size != 1)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "thread position chunk size applies only to thread "
                    "mapping");
  if (spmv == "wave-per-position" && reduction != "atomic")
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "thread position reduction applies only to thread "
                    "mapping");
  if (o->spmm_position_chunk_size < 1)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "thread position chunk size must be positive, but got "
                    "%lld",
                    (long long)o->spmm_position_chunk_size);
  if (!is_pow2(o->spmv_lanes_per_row) || o->spmv_lanes_per_row > 64)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "spmv-lanes-per-row must be a power of two between 1 and "
                    "64, but got %lld",
                    (long long)o->spmv_lanes_per_row);
  int64_t ppl = o->spmv_positions_per_lane;
  if (ppl != 1 && ppl != 2 && ppl != 4 && ppl != 8 && ppl != 16)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "spmv-positions-per-lane must be 1, 2, 4, 8 or 16, but "
                    "got %lld",
                    (long long)ppl);
  if (!is_pow2(o->spmm_lanes_per_row) || o->spmm_lanes_per_row > 64)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "spmm-lanes-per-row must be a power of two between 1 and "
                    "64, but got %lld",
                    (long long)o->spmm_lanes_per_row);
  int64_t sppl = o->spmm_positions_per_lane;
  if (sppl != 1 && sppl != 2 && sppl != 4 && sppl != 8 && sppl != 16)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "spmm-positions-per-lane must be 1, 2, 4, 8 or 16, but "
                    "got %lld",
                    (long long)sppl);
  if (o->bsr_use_mfma != 0 && o->bsr_use_mfma != 1)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "bsr-use-mfma must be 0 or 1, but got %lld",
                    (long long)o->bsr_use_mfma);
  if (o->sddmm_lanes_per_row != 1 && o->sddmm_lanes_per_row != 64)
    return sw::fail(SW_ERR_INVALID_OPTION,
                    "sddmm-lanes-per-row must be 1 or 64, but got %lld",
                    (long long)o->sddmm_lanes_per_row);
  return SW_OK;
}

const char *sw_last_error(void) { return g_last_error.c_str(); }

const char *sw_version(void) { return "sparsewave-amd 0.1 gfx950 wave64"; }

} // extern "C"
