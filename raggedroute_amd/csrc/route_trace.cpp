// Route-trace reader: the `.rrtrace` text format v1 of reference
// include/raggedroute/benchmark/adapter_utils.h:250-322 (load_route_trace_frame)
// and configs/workloads/route_trace.schema.json.
//
//   raggedroute.route_trace.v1          schema line, exact
//   <trace_id>                          [A-Za-z0-9._-]+
//   <source_kind>                       production | captured | synthetic_fixture
//   <tokens> <experts> <top_k> <frames>
//   <frame_id> <tokens * top_k expert ids>      one record per frame
//
// The whole file is validated whatever frame is requested: unique portable
// frame ids, every id in [0, experts), no expert repeated inside a token, no
// trailing data. Host code only (the ids feed the device entries afterwards).
#include <algorithm>
#include <cctype>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <set>
#include <string>
#include <vector>

#include "common.h"

namespace rr {
namespace {

bool portable_id(const std::string& value) noexcept {
  if (value.empty()) return false;
  for (const char c : value) {
    const auto byte = static_cast<unsigned char>(c);
    if (std::isalnum(byte) == 0 && c != '.' && c != '_' && c != '-') return false;
  }
  return true;
}

void copy_field(char* dst, std::size_t capacity, const std::string& src) noexcept {
  const std::size_t n = src.size() < capacity - 1 ? src.size() : capacity - 1;
  std::memcpy(dst, src.data(), n);
  dst[n] = '\0';
}

rr_status read_trace(const char* path, int32_t frame, rr_route_trace_info* info, int32_t* ids_out,
                     std::size_t capacity) {
  if (path == nullptr || path[0] == '\0' || frame < 0 || info == nullptr) {
    return invalid_argument("route_trace_path and route_trace_frame are invalid");
  }
  std::ifstream input(path);
  if (!input) return invalid_argument("cannot open route trace");
  std::string schema, trace_id, source_kind;
  int32_t tokens = 0, experts = 0, top_k = 0, frames = 0;
  if (!std::getline(input, schema) || schema != "raggedroute.route_trace.v1" ||
      !std::getline(input, trace_id) || !std::getline(input, source_kind) ||
      !(input >> tokens >> experts >> top_k >> frames)) {
    return invalid_argument("invalid route trace header");
  }
  if (!portable_id(trace_id) ||
      (source_kind != "production" && source_kind != "captured" &&
       source_kind != "synthetic_fixture") ||
      tokens < 1 || experts < 1 || experts > RR_MAX_EXPERTS || top_k < 1 || top_k > experts ||
      frames < 1 || frame >= frames) {
    return invalid_argument("invalid route trace metadata");
  }
  if (tokens > INT32_MAX / top_k) return invalid_argument("route trace route count exceeds int32");
  const std::size_t routes = static_cast<std::size_t>(tokens) * static_cast<std::size_t>(top_k);
  if (ids_out != nullptr && capacity < routes) {
    return invalid_argument("route trace frame does not fit the id buffer");
  }
  std::set<std::string> seen;
  std::vector<int32_t> ids(routes);
  std::vector<int32_t> token_ids(static_cast<std::size_t>(top_k));
  std::string selected_id;
  std::vector<int32_t> selected;  // handed out only once the whole file is valid
  for (int32_t f = 0; f < frames; ++f) {
    std::string frame_id;
    if (!(input >> frame_id) || !portable_id(frame_id) || !seen.insert(frame_id).second) {
      return invalid_argument("route trace frame id is invalid or duplicated");
    }
    for (std::size_t r = 0; r < routes; ++r) {
      if (!(input >> ids[r]) || ids[r] < 0 || ids[r] >= experts) {
        return invalid_argument("route trace contains an invalid expert id");
      }
    }
    // distinct experts inside each token (top_k <= 1024: a sorted copy per token)
    for (int32_t t = 0; t < tokens; ++t) {
      const int32_t* row = ids.data() + static_cast<std::size_t>(t) * top_k;
      token_ids.assign(row, row + top_k);
      std::sort(token_ids.begin(), token_ids.end());
      for (int32_t j = 1; j < top_k; ++j) {
        if (token_ids[static_cast<std::size_t>(j)] == token_ids[static_cast<std::size_t>(j - 1)]) {
          return invalid_argument("route trace repeats an expert within one token");
        }
      }
    }
    if (f == frame) {
      selected_id = frame_id;
      if (ids_out != nullptr) selected = ids;
    }
  }
  std::string trailing;
  if (input >> trailing) return invalid_argument("route trace has trailing data");
  if (ids_out != nullptr) std::memcpy(ids_out, selected.data(), routes * sizeof(int32_t));
  info->tokens = tokens;
  info->experts = experts;
  info->top_k = top_k;
  info->frame_count = frames;
  copy_field(info->trace_id, sizeof(info->trace_id), trace_id);
  copy_field(info->source_kind, sizeof(info->source_kind), source_kind);
  copy_field(info->frame_id, sizeof(info->frame_id), selected_id);
  return ok_status();
}

}  // namespace
}  // namespace rr

extern "C" rr_status rr_route_trace_read(const char* path, int32_t frame, rr_route_trace_info* info,
                                         int32_t* expert_ids, size_t capacity) {
  try {
    return rr::read_trace(path, frame, info, expert_ids, capacity);
  } catch (...) {  // allocation failure on a huge header: no exception crosses the C ABI
    return rr::invalid_argument("route trace could not be read");
  }
}
