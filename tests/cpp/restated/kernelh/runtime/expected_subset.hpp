// Test-only: the part of C++23 std::expected that the Backend binding uses,
// for C++ libraries that do not ship <expected> (GCC 11's, in this image).
// Included by runtime_error.hpp only when <expected> is missing; with a
// C++23 library the binding compiles against the real one. Covered:
// construction from a value or in place from an error (std::unexpect),
// has_value / operator bool, operator* / operator->, value(), error().
// std::unexpected is left out: GCC 11 still declares the pre-C++17
// function of that name, so the binding builds its errors with
// std::unexpect instead.
#ifndef KH_EXPECTED_SUBSET_HPP
#define KH_EXPECTED_SUBSET_HPP

#include <new>
#include <stdexcept>
#include <type_traits>
#include <utility>

namespace std {

struct unexpect_t {
  explicit unexpect_t() = default;
};
inline constexpr unexpect_t unexpect{};

template <class T, class E>
class expected {
 public:
  template <class U = T, class = enable_if_t<is_constructible_v<T, U &&>>>
  expected(U &&v) : ok_(true) {  // NOLINT: implicit, as in C++23
    new (&u_.v) T(std::forward<U>(v));
  }
  template <class... A>
  explicit expected(unexpect_t, A &&...a) : ok_(false) {
    new (&u_.e) E(std::forward<A>(a)...);
  }
  expected(expected &&o) : ok_(o.ok_) {
    if (ok_) new (&u_.v) T(std::move(o.u_.v));
    else new (&u_.e) E(std::move(o.u_.e));
  }
  expected(const expected &o) : ok_(o.ok_) {
    if (ok_) new (&u_.v) T(o.u_.v);
    else new (&u_.e) E(o.u_.e);
  }
  expected &operator=(const expected &) = delete;
  ~expected() {
    if (ok_) u_.v.~T();
    else u_.e.~E();
  }
  bool has_value() const { return ok_; }
  explicit operator bool() const { return ok_; }
  T &operator*() & { return u_.v; }
  const T &operator*() const & { return u_.v; }
  T &&operator*() && { return std::move(u_.v); }
  T *operator->() { return &u_.v; }
  const T *operator->() const { return &u_.v; }
  T &value() & {
    if (!ok_) throw logic_error("bad expected access");
    return u_.v;
  }
  const E &error() const & { return u_.e; }
  E &error() & { return u_.e; }

 private:
  union U {
    U() {}
    ~U() {}
    T v;
    E e;
  } u_;
  bool ok_;
};

template <class E>
class expected<void, E> {
 public:
  expected() = default;
  template <class... A>
  explicit expected(unexpect_t, A &&...a) : ok_(false), e_(std::forward<A>(a)...) {}
  bool has_value() const { return ok_; }
  explicit operator bool() const { return ok_; }
  void value() const {
    if (!ok_) throw logic_error("bad expected access");
  }
  const E &error() const & { return e_; }
  E &error() & { return e_; }

 private:
  bool ok_ = true;
  E e_{};
};

}  // namespace std

#endif
