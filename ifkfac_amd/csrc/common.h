// Shared device/host helpers for the IFKFAC curvature kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this library:
//   * all matrices are row-major; element (i, j) of a matrix with leading
//   * dimension ld lives at ptr[i * ld + j];
//   * accumulation is always fp32; bf16 values are produced with
//     round-to-nearest-even, the rounding torch's `.to(torch.bfloat16)` uses;
//   * every launch goes to the caller's stream; nothing here synchronises
//     the device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

namespace ifk {

typedef uint16_t bf16_t;  // raw bf16 bits

enum DType { DT_F32 = 0, DT_BF16 = 1 };
enum Math { MATH_F32 = 0, MATH_BF16 = 1 };

// Triangular structure flags for GEMM operands (what op(X) is known to be).
enum Tri { TRI_NONE = 0, TRI_UPPER = 1, TRI_LOWER = 2 };

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (bit-exact RNE, NaN-preserving)
// ---------------------------------------------------------------------------
__host__ __device__ inline bf16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    return (bf16_t)((u >> 16) | 0x0040u);  // quiet NaN, keep sign/payload top
  }
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (bf16_t)(u >> 16);
}

__host__ __device__ inline float bf16_to_f32(bf16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Pack two floats into one dword of two RNE bf16 values (lo in bits 0..15).
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

template <int DT> struct Elem;
template <> struct Elem<DT_F32> {
  typedef float T;
  __device__ static inline float load(const float* p) { return *p; }
  __device__ static inline void store(float* p, float v) { *p = v; }
};
template <> struct Elem<DT_BF16> {
  typedef bf16_t T;
  __device__ static inline float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ static inline void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

// ---------------------------------------------------------------------------
// Error reporting (host side): thread-local last-error string.
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
const char* get_error();

struct Status {
  int code;
  static Status ok() { return Status{0}; }
};

#define IFK_OK 0
#define IFK_ERR_INVALID (-1)
#define IFK_ERR_WORKSPACE (-2)
#define IFK_ERR_HIP (-3)

// Returns IFK_ERR_HIP (with message) if the last launch failed.
int check_launch(const char* what);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// A bump allocator over a caller-provided workspace.  Never allocates device
// memory itself; running out is reported, not hidden.  With base == nullptr it
// only measures: take() returns nullptr and `used` accumulates the size the
// same plan needs, which is how the *_workspace_size entry points answer.
struct Arena {
  char* base;
  size_t cap;
  size_t used;
  bool overflow;
  Arena(void* p, size_t c) : base((char*)p), cap(c), used(0), overflow(false) {}
  bool measuring() const { return base == nullptr; }
  template <typename T> T* take(size_t count) {
    size_t off = align_up(used, 256);
    size_t bytes = align_up(count * sizeof(T), 256);
    used = off + bytes;
    if (base == nullptr) return nullptr;
    if (used > cap) {
      overflow = true;
      return nullptr;
    }
    return (T*)(base + off);
  }
};

}  // namespace ifk
