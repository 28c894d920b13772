// Node pointer aliases (reference autograd/IntrusivePtr.hpp:15-19).
#pragma once

#include <memory>

namespace tensorforge {

template <typename T>
using NodePtr = std::shared_ptr<T>;
template <typename T>
using WeakNodePtr = std::weak_ptr<T>;

}  // namespace tensorforge
