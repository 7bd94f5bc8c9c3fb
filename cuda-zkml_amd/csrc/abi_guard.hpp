// Exception guard for the host-only C entry points (no device code): a C++
// exception, a failed host allocation mostly, becomes a status instead of
// crossing the C ABI.
#pragma once
#include <new>

#include "../../include/zkml_gpu.h"

namespace zkh {

template <class Fn>
int abi_guard(Fn&& fn) noexcept {
  try {
    return fn();
  } catch (const std::bad_alloc&) {
    return ZK_ERR_OOM;
  } catch (...) {
    return ZK_ERR_INVALID;
  }
}

}  // namespace zkh
