// Option cursor for the kernelh subcommands. It walks the words after the
// subcommand once; each call offers the current word to one option and
// consumes it (and its value) on a match, so a subcommand reads as a chain
// of `if (a.value("--out", out)) ... else if (a.flag("--occupancy")) ...`
// ending in an "unknown option" branch for the word `a.word()`.
//
// Options take their value as the next word or after '=' ("--out d" or
// "--out=d"), as the reference's CLI accepts them (tools/kernelh/main.cpp).
// A value option that ends the command line is a usage error: reported on
// stderr as "error: <option> requires a value", exit status 2.
#pragma once

#include <charconv>
#include <cstdlib>
#include <iostream>
#include <string>
#include <string_view>
#include <vector>

namespace khcli {

class ArgCursor {
 public:
  ArgCursor(int argc, char **argv, int first) {
    for (int i = first; i < argc; ++i) words_.emplace_back(argv[i]);
  }

  bool done() const { return at_ >= words_.size(); }
  const std::string &word() const { return words_[at_]; }
  // Skips the current word (after the caller has dealt with it).
  void skip() { ++at_; }

  // A switch: "--name".
  bool flag(std::string_view name) {
    if (done() || word() != name) return false;
    ++at_;
    return true;
  }

  // "--name value" or "--name=value".
  bool value(std::string_view name, std::string &out) {
    if (done()) return false;
    const std::string &w = word();
    if (w.size() > name.size() && w.compare(0, name.size(), name) == 0 && w[name.size()] == '=') {
      out = w.substr(name.size() + 1);
      ++at_;
      return true;
    }
    if (w != name) return false;
    if (at_ + 1 >= words_.size()) {
      std::cerr << "error: " << name << " requires a value\n";
      std::exit(2);
    }
    out = words_[at_ + 1];
    at_ += 2;
    return true;
  }

  // An integer option within [lo, hi]. On a match whose value is not such
  // an integer, `ok` becomes false after "error: <name> must be an integer
  // in [lo,hi]" on stderr; the caller exits with status 2.
  bool integer(std::string_view name, long lo, long hi, long &out, bool &ok) {
    std::string text;
    if (!value(name, text)) return false;
    long v = 0;
    const char *first = text.data(), *last = text.data() + text.size();
    const auto [end, ec] = std::from_chars(first, last, v);
    if (ec != std::errc() || end != last || first == last || v < lo || v > hi) {
      std::cerr << "error: " << name << " must be an integer in [" << lo << "," << hi << "]\n";
      ok = false;
      return true;
    }
    out = v;
    return true;
  }

 private:
  std::vector<std::string> words_;
  size_t at_ = 0;
};

}  // namespace khcli
