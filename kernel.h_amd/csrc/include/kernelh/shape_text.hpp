// Shape text: the `--shape` syntax of the kernelh CLI and of the runtime's
// launcher queries (khrt_template_geometry and friends), one parser for both.
//
// Grammar (the interface the reference's CLI and bench accept,
// tools/kernelh/main.cpp:242-266, bench/harness/shape_text.cpp:19-44):
//     shape := dim ( ',' dim )*
//     dim   := name '=' integer
//     name  := one or more characters other than '=' and ','
//     integer := optional sign, then decimal digits, within int64
// A later dim of the same name replaces an earlier one. Nothing else is
// accepted: no empty text, empty names or values, trailing commas, or
// characters after the digits.
//
// Written as a single left-to-right scan with a cursor; std::from_chars does
// the integer conversion (no locale, no errno, no leading whitespace).
#pragma once

#include <charconv>
#include <cstdint>
#include <map>
#include <string>
#include <string_view>

namespace kernelh {

using ShapeDims = std::map<std::string, int64_t>;

// Parses `text` into `dims` (added to what it holds). On failure returns
// false and, when `why` is given, says what was expected and where.
inline bool parse_shape_text(std::string_view text, ShapeDims &dims, std::string *why = nullptr) {
  size_t at = 0;
  auto reject = [&](const char *expected) {
    if (why != nullptr) *why = std::string(expected) + " at offset " + std::to_string(at) + " of '" +
                               std::string(text) + "'";
    return false;
  };
  if (text.empty()) return reject("a dimension");
  for (;;) {
    const size_t name_at = at;
    while (at < text.size() && text[at] != '=' && text[at] != ',') ++at;
    if (at == name_at) return reject("a dimension name");
    if (at == text.size() || text[at] != '=') return reject("'=' after the dimension name");
    const std::string_view name = text.substr(name_at, at - name_at);
    ++at;
    const char *first = text.data() + at, *last = text.data() + text.size();
    if (first != last && *first == '+') {  // from_chars takes '-' only
      ++first;
      if (first != last && *first == '-') return reject("a decimal integer in int64 range");
    }
    int64_t value = 0;
    const auto [end, ec] = std::from_chars(first, last, value);
    if (ec != std::errc() || end == first) return reject("a decimal integer in int64 range");
    at = static_cast<size_t>(end - text.data());
    dims[std::string(name)] = value;
    if (at == text.size()) return true;
    if (text[at] != ',') return reject("',' or the end after the integer");
    ++at;
  }
}

}  // namespace kernelh
