// Scope guard: runs a callable when the enclosing scope ends, normally or by an exception, unless
// released first.  Host code only; no HIP dependency (tested alone by tests/test_scope.py).
#pragma once

#include <utility>

namespace laya {

template <typename F>
class ScopeExit {
 public:
  explicit ScopeExit(F f) : f_(std::move(f)) {}
  ScopeExit(const ScopeExit&) = delete;
  ScopeExit& operator=(const ScopeExit&) = delete;
  ~ScopeExit() {
    if (armed_) f_();
  }
  void release() { armed_ = false; }

 private:
  F f_;
  bool armed_ = true;
};

}  // namespace laya
