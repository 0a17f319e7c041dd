// expected.hpp — std::expected where the standard library has it, otherwise a
// small replacement with the subset of its interface the engine uses.
//
// The reference engine returns std::expected<T, std::error_code> everywhere
// (e.g. include/backend.hpp:9). libstdc++ 11 (the library of both g++ 11 and
// ROCm clang on this platform) ships no <expected>, so the engine spells the
// type infer::expected / infer::unexpected and this header maps the names.
#pragma once

#if defined(__has_include)
#if __has_include(<expected>) && __cplusplus > 202002L
#include <expected>
#endif
#endif

#include <system_error>
#include <type_traits>
#include <utility>
#include <variant>

namespace infer {

#if defined(__cpp_lib_expected)

template <class T, class E>
using expected = std::expected<T, E>;
template <class E>
using unexpected = std::unexpected<E>;

#else

template <class E>
class unexpected {
 public:
  explicit unexpected(E e) : e_(std::move(e)) {}
  const E &error() const & { return e_; }
  E &error() & { return e_; }
  E &&error() && { return std::move(e_); }

 private:
  E e_;
};
template <class E>
unexpected(E) -> unexpected<E>;

namespace detail {
template <class E>
struct err_box {
  E e;
};
}  // namespace detail

template <class T, class E>
class expected {
 public:
  using value_type = T;
  using error_type = E;

  expected() : v_(std::in_place_index<0>) {}
  template <class U = T,
            std::enable_if_t<std::is_constructible_v<T, U &&> &&
                                 !std::is_same_v<std::decay_t<U>, expected> &&
                                 !std::is_same_v<std::decay_t<U>, unexpected<E>>,
                             int> = 0>
  expected(U &&v) : v_(std::in_place_index<0>, std::forward<U>(v)) {}
  template <class G>
  expected(const unexpected<G> &u) : v_(std::in_place_index<1>, detail::err_box<E>{E(u.error())}) {}
  template <class G>
  expected(unexpected<G> &&u)
      : v_(std::in_place_index<1>, detail::err_box<E>{E(std::move(u).error())}) {}

  bool has_value() const noexcept { return v_.index() == 0; }
  explicit operator bool() const noexcept { return has_value(); }

  T &value() & { return std::get<0>(v_); }
  const T &value() const & { return std::get<0>(v_); }
  T &&value() && { return std::get<0>(std::move(v_)); }
  T &operator*() & { return std::get<0>(v_); }
  const T &operator*() const & { return std::get<0>(v_); }
  T &&operator*() && { return std::get<0>(std::move(v_)); }
  T *operator->() { return &std::get<0>(v_); }
  const T *operator->() const { return &std::get<0>(v_); }

  const E &error() const & { return std::get<1>(v_).e; }
  E &error() & { return std::get<1>(v_).e; }

 private:
  std::variant<T, detail::err_box<E>> v_;
};

template <class E>
class expected<void, E> {
 public:
  using value_type = void;
  using error_type = E;

  expected() = default;
  template <class G>
  expected(const unexpected<G> &u) : ok_(false), e_(E(u.error())) {}
  template <class G>
  expected(unexpected<G> &&u) : ok_(false), e_(E(std::move(u).error())) {}

  bool has_value() const noexcept { return ok_; }
  explicit operator bool() const noexcept { return ok_; }
  void value() const {}
  void operator*() const {}
  const E &error() const & { return e_; }

 private:
  bool ok_ = true;
  E e_{};
};

#endif

using std::error_code;

inline unexpected<std::error_code> fail(std::errc e) {
  return unexpected<std::error_code>(std::make_error_code(e));
}

}  // namespace infer
