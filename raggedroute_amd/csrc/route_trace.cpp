// Route traces: reader of the `.rrtrace` text format v1, the normalised text
// form of a `raggedroute.route_trace.v1` document (reference
// configs/workloads/route_trace.schema.json; reference
// configs/workloads/synthetic_fixture.rrtrace is one such file). Layout:
//
//   line 1   raggedroute.route_trace.v1
//   line 2   trace id        letters, digits, '.', '_', '-'
//   line 3   source kind     production | captured | synthetic_fixture
//   line 4   T E top_k F     four integers
//   then     F frame records, each a frame id (same alphabet as the trace id)
//            followed by T * top_k expert ids, token-major
//
// The file is read into memory once and scanned by a cursor: the four header
// lines are taken as whole lines (a trailing CR is dropped), the records as a
// stream of whitespace-separated words, so a record may wrap lines. Every
// record is checked, whichever frame is asked for; the asked frame is staged
// and reaches the caller's buffer only once the last record and the end of
// the file have checked out. A token that names one expert twice is caught
// with a stamp per expert (the number of the token that used it last):
// O(top_k) per token. E is capped at RR_MAX_EXPERTS (the schema's cap is 64).
// Host code only; messages are static strings.
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_set>
#include <vector>

#include "common.h"

namespace rr {
namespace {

constexpr const char* kSchemaTag = "raggedroute.route_trace.v1";

bool id_char(char c) noexcept {
  return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') || c == '.' ||
         c == '_' || c == '-';
}

bool is_identifier(const std::string& s) noexcept {
  if (s.empty()) return false;
  for (const char c : s) {
    if (!id_char(c)) return false;
  }
  return true;
}

bool is_space(char c) noexcept { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\v' || c == '\f'; }

// Whole decimal integer in int32 range (optional sign, nothing else).
bool parse_int32(const std::string& word, int32_t* out) noexcept {
  if (word.empty()) return false;
  errno = 0;
  char* end = nullptr;
  const long long v = std::strtoll(word.c_str(), &end, 10);
  if (errno != 0 || end != word.c_str() + word.size()) return false;
  if (v < INT32_MIN || v > INT32_MAX) return false;
  *out = static_cast<int32_t>(v);
  return true;
}

class Cursor {
 public:
  explicit Cursor(std::string text) : text_(std::move(text)) {}

  // Next line without its terminator (and without a trailing CR); false at the end.
  bool line(std::string* out) {
    if (at_ >= text_.size()) return false;
    std::size_t stop = text_.find('\n', at_);
    if (stop == std::string::npos) stop = text_.size();
    std::size_t last = stop;
    if (last > at_ && text_[last - 1] == '\r') --last;
    out->assign(text_, at_, last - at_);
    at_ = stop < text_.size() ? stop + 1 : stop;
    return true;
  }

  // Next whitespace-separated word; false when only whitespace is left.
  bool word(std::string* out) {
    while (at_ < text_.size() && is_space(text_[at_])) ++at_;
    if (at_ >= text_.size()) return false;
    const std::size_t begin = at_;
    while (at_ < text_.size() && !is_space(text_[at_])) ++at_;
    out->assign(text_, begin, at_ - begin);
    return true;
  }

 private:
  std::string text_;
  std::size_t at_ = 0;
};

bool slurp(const char* path, std::string* text) {
  std::FILE* file = std::fopen(path, "rb");
  if (file == nullptr) return false;
  char block[1 << 16];
  std::size_t got = 0;
  while ((got = std::fread(block, 1, sizeof(block), file)) > 0) text->append(block, got);
  const bool failed = std::ferror(file) != 0;
  std::fclose(file);
  return !failed;
}

void set_text(char* dst, std::size_t size, const std::string& src) noexcept {
  const std::size_t n = src.size() < size ? src.size() : size - 1;
  std::memcpy(dst, src.data(), n);
  dst[n] = '\0';
}

rr_status load(const char* path, int32_t want, rr_route_trace_info* info, int32_t* ids_out,
               std::size_t capacity) {
  if (path == nullptr || path[0] == '\0' || want < 0 || info == nullptr) {
    return invalid_argument("rr_route_trace_read needs a path, a frame index >= 0 and an info struct");
  }
  std::string text;
  if (!slurp(path, &text)) return invalid_argument("route trace file cannot be opened or read");
  Cursor cur(std::move(text));

  std::string tag, trace_id, kind;
  if (!cur.line(&tag) || tag != kSchemaTag) {
    return invalid_argument("route trace: line 1 must be raggedroute.route_trace.v1");
  }
  if (!cur.line(&trace_id) || !is_identifier(trace_id)) {
    return invalid_argument("route trace: line 2 (trace id) is not a portable identifier");
  }
  if (!cur.line(&kind) || (kind != "production" && kind != "captured" && kind != "synthetic_fixture")) {
    return invalid_argument("route trace: line 3 names no known source kind");
  }
  // The shape is the next four words, wherever the lines break (as the
  // reference reads it with stream extraction); the first record may follow
  // on the same line.
  int32_t shape[4] = {0, 0, 0, 0};
  for (int32_t& v : shape) {
    std::string w;
    if (!cur.word(&w) || !parse_int32(w, &v)) {
      return invalid_argument("route trace: the shape after line 3 must be four integers T E top_k frames");
    }
  }
  const int32_t tokens = shape[0], experts = shape[1], top_k = shape[2], frames = shape[3];
  if (tokens < 1 || experts < 1 || experts > RR_MAX_EXPERTS || top_k < 1 || top_k > experts ||
      frames < 1) {
    return invalid_argument("route trace: shape out of range (T >= 1, 1 <= top_k <= E <= 1024, frames >= 1)");
  }
  if (tokens > INT32_MAX / top_k) return invalid_argument("route trace: T * top_k exceeds int32 indexing");
  if (want >= frames) return invalid_argument("route trace: frame index past the last frame");
  const std::size_t routes = static_cast<std::size_t>(tokens) * static_cast<std::size_t>(top_k);
  if (ids_out != nullptr && capacity < routes) {
    return invalid_argument("route trace: the id buffer holds fewer than T * top_k ids");
  }

  std::unordered_set<std::string> frame_ids;
  std::vector<int32_t> staged;  // the asked frame, handed out at the end
  std::vector<int64_t> stamp(static_cast<std::size_t>(experts), -1);
  std::string selected_name, w;
  int64_t token_number = 0;  // over every token of every frame
  for (int32_t f = 0; f < frames; ++f) {
    std::string name;
    if (!cur.word(&name) || !is_identifier(name)) {
      return invalid_argument("route trace: a frame record lacks a portable frame id");
    }
    if (!frame_ids.insert(name).second) return invalid_argument("route trace: two frames share a frame id");
    const bool keep = f == want;
    if (keep) {
      selected_name = name;
      if (ids_out != nullptr) staged.resize(routes);
    }
    for (int32_t t = 0; t < tokens; ++t, ++token_number) {
      for (int32_t j = 0; j < top_k; ++j) {
        int32_t id = 0;
        if (!cur.word(&w) || !parse_int32(w, &id)) {
          return invalid_argument("route trace: a frame record ends early or holds a non-integer");
        }
        if (id < 0 || id >= experts) return invalid_argument("route trace: an expert id lies outside [0, E)");
        int64_t& last = stamp[static_cast<std::size_t>(id)];
        if (last == token_number) return invalid_argument("route trace: a token names one expert twice");
        last = token_number;
        if (keep && ids_out != nullptr) {
          staged[static_cast<std::size_t>(t) * top_k + j] = id;
        }
      }
    }
  }
  if (cur.word(&w)) return invalid_argument("route trace: text follows the last frame record");

  if (ids_out != nullptr) std::memcpy(ids_out, staged.data(), routes * sizeof(int32_t));
  info->tokens = tokens;
  info->experts = experts;
  info->top_k = top_k;
  info->frame_count = frames;
  set_text(info->trace_id, sizeof(info->trace_id), trace_id);
  set_text(info->source_kind, sizeof(info->source_kind), kind);
  set_text(info->frame_id, sizeof(info->frame_id), selected_name);
  return ok_status();
}

}  // namespace
}  // namespace rr

extern "C" rr_status rr_route_trace_read(const char* path, int32_t frame, rr_route_trace_info* info,
                                         int32_t* expert_ids, size_t capacity) {
  try {
    return rr::load(path, frame, info, expert_ids, capacity);
  } catch (...) {  // (allocation failure on a huge file: nothing crosses the C ABI)
    return rr::invalid_argument("route trace: out of host memory while reading");
  }
}
