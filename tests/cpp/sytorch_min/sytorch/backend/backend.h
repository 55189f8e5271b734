// Minimal sytorch declarations for compiling include/mpcx_sytorch.hpp in the
// tests: the tensor types and the Backend<T> virtual interface that the
// reference's backends override (gpu_mpc/ddg_orca_base.h:37-322,
// gpu_mpc/ddg_orca.h:30-139; `sub` is the method the reference's patch adds to
// Backend, patches/EzPC-GPU-MPC.track3.patch:1-13), reconstructed from those
// call sites.  sytorch itself (EzPC) is not part of the reference.
#pragma once
#include <cstdint>
#include <cstdlib>
#include <functional>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

typedef uint8_t u8;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int64_t i64;
#define MPCX_EZPC_HAVE_INT_TYPES 1

template <typename T>
class Tensor1D {
 public:
  T *data = nullptr;
  T *d_data = nullptr;
  u64 d1 = 0;
  explicit Tensor1D(u64 n) : d1(n) { data = new T[n](); }
  ~Tensor1D() { delete[] data; }
  Tensor1D(const Tensor1D &) = delete;
  Tensor1D &operator=(const Tensor1D &) = delete;
  u64 size() const { return d1; }
};

// A view: host data and device data with two dimensions.
template <typename T>
class Tensor2D {
 public:
  T *data = nullptr;
  T *d_data = nullptr;
  u64 d1 = 0, d2 = 0;
  Tensor2D(T *data_, T *d_data_, u64 d1_, u64 d2_) : data(data_), d_data(d_data_), d1(d1_), d2(d2_) {}
  u64 size() const { return d1 * d2; }
};

template <typename T>
class Tensor4D {
 public:
  T *data = nullptr;
  T *d_data = nullptr;
  u64 d1 = 0, d2 = 0, d3 = 0, d4 = 0;
  u64 size() const { return d1 * d2 * d3 * d4; }
};

template <typename T>
class Tensor {
 public:
  T *data = nullptr;    // host
  T *d_data = nullptr;  // device
  std::vector<u64> shape;
  explicit Tensor(const std::vector<u64> &s) : shape(s) { data = new T[size()](); }
  // a view of existing host and device arrays (masked_maxpool_layer.h:96, 109)
  Tensor(T *data_, T *d_data_, const std::vector<u64> &s) : data(data_), d_data(d_data_), shape(s), owns_(false) {}
  ~Tensor() {
    if (owns_) delete[] data;
  }
  Tensor(const Tensor &) = delete;
  Tensor &operator=(const Tensor &) = delete;
  u64 size() const {
    u64 n = 1;
    for (u64 d : shape) n *= d;
    return n;
  }
  bool is_same_shape(const Tensor<T> &o) const { return shape == o.shape; }
  Tensor2D<T> as_2d() const {
    const u64 d2 = shape.empty() ? 1 : shape.back();
    return Tensor2D<T>(data, d_data, size() / d2, d2);
  }

 private:
  bool owns_ = true;
};

template <typename T>
struct LayerGraphNode {
  std::vector<LayerGraphNode<T> *> children;
};

template <typename T>
void topologicalApply(LayerGraphNode<T> *root, std::function<void(LayerGraphNode<T> *, LayerGraphNode<T> *)> fn) {
  std::set<LayerGraphNode<T> *> seen;
  std::vector<LayerGraphNode<T> *> st{root};
  while (!st.empty()) {
    LayerGraphNode<T> *n = st.back();
    st.pop_back();
    if (!n || !seen.insert(n).second) continue;
    fn(n, root);
    for (auto *c : n->children) st.push_back(c);
  }
}

template <typename T>
class Backend {
 public:
  virtual ~Backend() = default;
  virtual void matmul(const Tensor2D<T> &a, const Tensor2D<T> &b, Tensor2D<T> &c) { nope("matmul"); }
  virtual void matmul(const Tensor2D<T> &a, const Tensor2D<T> &b, Tensor2D<T> &c, bool useBias, Tensor1D<T> &d,
                      bool isFirst) {
    nope("matmul");
  }
  virtual void mul(const Tensor<T> &a, const Tensor<T> &b, Tensor<T> &out) { nope("mul"); }
  virtual void scalarmul(Tensor<T> &x, T scalar, Tensor<T> &y) { nope("scalarmul"); }
  virtual void sub(Tensor<T> &b, Tensor<T> &a, Tensor<T> &out) { nope("sub"); }
  virtual void add(const std::vector<Tensor<T> *> &in, Tensor<T> &out) { nope("add"); }
  virtual void relu(Tensor<T> &in, Tensor<T> &out, const Tensor<T> &drelu, u64 scale, int mode) { nope("relu"); }
  virtual void truncateForward(Tensor<T> &in, u64 shift, u8 mode = 0) { nope("truncateForward"); }
  virtual void signext(Tensor<T> &x, u64 scale) { nope("signext"); }
  virtual void output(Tensor<T> &a) { nope("output"); }
  virtual void optimize(LayerGraphNode<T> *root) {}

 protected:
  [[noreturn]] static void nope(const char *what) { throw std::runtime_error(std::string(what) + " not implemented"); }
};
