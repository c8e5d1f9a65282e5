// Host emulation of the HIP device subset the lps kernels use: test
// infrastructure only (tests/test_hostemu.py), never part of the product.
//
// The kernel sources are compiled unchanged for x86 with clang
// (-fsanitize=address,undefined -fsanitize=bounds): this header stands in for
// <hip/hip_runtime.h>.  A launch runs its blocks one after another; a block's
// threads are host threads.  Wave-level operations (ballots, DPP lane moves,
// readlane, shuffles) exchange values through a per-wave buffer between two
// wave barriers, so every lane of a wave must reach them together, as wave-
// uniform control flow on the GPU guarantees.  Lanes that have returned are
// out of every barrier and ballot (as inactive lanes are on the GPU).  A
// barrier that waits longer than LPS_EMU_BARRIER_TIMEOUT_S reports a deadlock
// (divergent barriers or lane operations) and aborts.
//
// Because blocks run one at a time, `__shared__` variables are statics, and a
// kernel that waits for another block of its launch would time out: only
// launches whose blocks never wait for each other are emulated (row-group
// plans of one chunk per row, the streaming and general kernels).
#pragma once

#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#define LPS_HOST_EMU 1

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline __attribute__((always_inline))
#define __shared__ static
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) (&(x))
// the kernels' register-pinning hook (an AMDGPU VGPR constraint on the GPU)
#define LPS_KEEP_VGPR(x) __asm__ volatile("" : "+r"(x))

typedef int hipError_t;
typedef void* hipStream_t;
enum { hipSuccess = 0, hipErrorNotInitialized = 3, hipErrorInvalidValue = 1 };
enum { hipDeviceAttributeMultiprocessorCount = 0 };
enum { hipMemcpyDeviceToHost = 2 };

struct dim3 {
  uint32_t x, y, z;
  constexpr dim3(uint32_t a = 1, uint32_t b = 1, uint32_t c = 1) : x(a), y(b), z(c) {}
};
struct uint4 { uint32_t x, y, z, w; };
struct uint2 { uint32_t x, y; };
struct float2 { float x, y; };
inline uint4 make_uint4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return uint4{a, b, c, d}; }
inline float2 make_float2(float a, float b) { return float2{a, b}; }

template <typename T> inline T min(T a, T b) { return a < b ? a : b; }
template <typename T> inline T max(T a, T b) { return a > b ? a : b; }
inline int64_t min(int64_t a, int b) { return a < b ? a : b; }
inline int64_t min(int a, int64_t b) { return a < b ? a : b; }
inline int64_t max(int64_t a, int b) { return a > b ? a : b; }
inline int64_t max(int a, int64_t b) { return a > b ? a : b; }
inline uint32_t min(uint32_t a, int b) { return a < (uint32_t)b ? a : (uint32_t)b; }

namespace lps_emu {

#ifndef LPS_EMU_BARRIER_TIMEOUT_S
#define LPS_EMU_BARRIER_TIMEOUT_S 60
#endif

// Progress of every barrier (a watchdog aborts a run whose barriers stop).
inline std::atomic<uint64_t> g_progress{0};

// A barrier whose participants can leave (the GPU's barrier counts only the
// waves that have not ended).  Arrivals update a short critical section;
// waiters sleep on the generation word (a futex), so a release does not make
// every waiter contend for the lock.
struct Barrier {
  std::mutex m;
  std::atomic<uint32_t> gen{0};
  int expected = 0, arrived = 0;
  const char* what = "";
  void init(int n, const char* w) { expected = n; arrived = 0; what = w; }
  void release_locked() {
    arrived = 0;
    gen.fetch_add(1, std::memory_order_release);
    g_progress.fetch_add(1, std::memory_order_relaxed);
    gen.notify_all();
  }
  void wait() {
    uint32_t g;
    {
      std::lock_guard<std::mutex> l(m);
      g = gen.load(std::memory_order_relaxed);
      if (++arrived >= expected) { release_locked(); return; }
    }
    for (int i = 0; i < 64 && gen.load(std::memory_order_acquire) == g; i++) std::this_thread::yield();
    while (gen.load(std::memory_order_acquire) == g) gen.wait(g, std::memory_order_acquire);
  }
  void leave() {
    std::lock_guard<std::mutex> l(m);
    expected--;
    if (expected > 0 && arrived >= expected) release_locked();
  }
};

// Aborts the run when no barrier has been released for
// LPS_EMU_BARRIER_TIMEOUT_S seconds while a launch runs (divergent barriers
// or lane operations never complete).
inline std::atomic<int> g_launching{0};
inline void watchdog_start() {
  static std::once_flag once;
  std::call_once(once, [] {
    std::thread([] {
      uint64_t last = 0;
      int still = 0;
      for (;;) {
        std::this_thread::sleep_for(std::chrono::seconds(1));
        const uint64_t p = g_progress.load();
        if (g_launching.load() && p == last) {
          if (++still >= LPS_EMU_BARRIER_TIMEOUT_S) {
            fprintf(stderr, "hostemu: no barrier released for %d s: deadlock (divergent barriers or lane ops)\n",
                    LPS_EMU_BARRIER_TIMEOUT_S);
            abort();
          }
        } else {
          still = 0;
        }
        last = p;
      }
    }).detach();
  });
}

struct Wave {
  Barrier bar;
  uint64_t buf[64];
  uint64_t alive;  // lanes that have not returned
};

struct Block {
  Barrier bar;
  std::vector<Wave*> waves;
};

struct Tid {
  uint32_t x, y, z;
};
inline thread_local Tid t_thread{0, 0, 0};
inline thread_local Tid t_block{0, 0, 0};
inline thread_local Wave* t_wave = nullptr;
inline thread_local Block* t_blk = nullptr;
inline Tid g_bdim{1, 1, 1}, g_gdim{1, 1, 1};

inline int lane() { return (int)(t_thread.x & 63u); }

// Every lane publishes v, then computes its result from the wave's values.
template <typename T, typename F>
inline T xchg(T v, F f) {
  static_assert(sizeof(T) <= 8, "lane values of at most 8 bytes");
  Wave* w = t_wave;
  uint64_t b = 0;
  memcpy(&b, &v, sizeof(T));
  w->buf[lane()] = b;
  w->bar.wait();
  T r = f(w->buf, w->alive);
  w->bar.wait();
  return r;
}
template <typename T>
inline T from_bits(uint64_t b) {
  T v;
  memcpy(&v, &b, sizeof(T));
  return v;
}

inline void launch(dim3 grid, dim3 block, std::function<void()> body) {
  watchdog_start();
  g_launching.store(1);
  g_bdim = Tid{block.x, block.y, block.z};
  g_gdim = Tid{grid.x, grid.y, grid.z};
  const int nt = (int)(block.x * block.y * block.z);
  const int nw = (nt + 63) / 64;
  for (uint32_t bz = 0; bz < grid.z; bz++)
    for (uint32_t by = 0; by < grid.y; by++)
      for (uint32_t bx = 0; bx < grid.x; bx++) {
        Block B;
        B.bar.init(nt, "block");
        std::vector<Wave> waves(nw);
        for (int i = 0; i < nw; i++) {
          const int n = (i + 1) * 64 <= nt ? 64 : nt - i * 64;
          waves[i].bar.init(n, "wave");
          waves[i].alive = n == 64 ? ~0ull : ((1ull << n) - 1ull);
          B.waves.push_back(&waves[i]);
        }
        struct Arg {
          Block* B;
          std::function<void()>* body;
          Tid t, b;
        };
        std::vector<Arg> args(nt);
        std::vector<pthread_t> th(nt);
        pthread_attr_t at;
        pthread_attr_init(&at);
        pthread_attr_setstacksize(&at, 1 << 20);
        for (int t = 0; t < nt; t++) {
          args[t] = Arg{&B, &body, Tid{(uint32_t)t, 0, 0}, Tid{bx, by, bz}};
          auto run = [](void* p) -> void* {
            Arg* a = static_cast<Arg*>(p);
            t_thread = a->t;
            t_block = a->b;
            t_blk = a->B;
            t_wave = a->B->waves[a->t.x / 64];
            (*a->body)();
            // this lane ends: out of its wave's ballots and barriers, and the block's
            {
              std::lock_guard<std::mutex> l(t_wave->bar.m);
              t_wave->alive &= ~(1ull << (a->t.x & 63));
            }
            t_wave->bar.leave();
            t_blk->bar.leave();
            return nullptr;
          };
          if (pthread_create(&th[t], &at, run, &args[t]) != 0) {
            fprintf(stderr, "hostemu: pthread_create failed\n");
            abort();
          }
        }
        for (int t = 0; t < nt; t++) pthread_join(th[t], nullptr);
        pthread_attr_destroy(&at);
        g_progress.fetch_add(1, std::memory_order_relaxed);
      }
  g_launching.store(0);
}

// DPP lane move (GFX9 controls used by the kernels): quad_perm, row_shr:n,
// row_mirror, row_half_mirror, row_bcast:15, row_bcast:31.
inline int dpp_src(int l, int ctrl) {
  const int row = l & ~15, in = l & 15;
  if (ctrl <= 0xFF) return (l & ~3) + ((ctrl >> (2 * (l & 3))) & 3);
  if (ctrl >= 0x111 && ctrl <= 0x11F) {
    const int n = ctrl - 0x110;
    return in - n >= 0 ? l - n : -1;
  }
  if (ctrl >= 0x121 && ctrl <= 0x12F) return row + ((in - (ctrl - 0x120)) & 15);  // row_ror:n
  if (ctrl == 0x140) return row + 15 - in;
  if (ctrl == 0x141) return (l & ~7) + 7 - (l & 7);
  if (ctrl == 0x142) return row >= 16 ? row - 1 : -1;
  if (ctrl == 0x143) return row >= 32 ? 31 : -1;
  fprintf(stderr, "hostemu: unsupported DPP control 0x%x\n", ctrl);
  abort();
}

}  // namespace lps_emu

#define threadIdx (::lps_emu::t_thread)
#define blockIdx (::lps_emu::t_block)
#define blockDim (::lps_emu::g_bdim)
#define gridDim (::lps_emu::g_gdim)

inline void __syncthreads() { lps_emu::t_blk->bar.wait(); }

#define hipLaunchKernelGGL(K, G, B, SHM, STREAM, ...) ::lps_emu::launch(dim3(G), dim3(B), [=]() { K(__VA_ARGS__); })
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, int, int) { *v = 256; return hipSuccess; }
template <typename T>
inline hipError_t hipGetSymbolAddress(void** p, T* sym) { *p = (void*)sym; return hipSuccess; }
inline hipError_t hipMemsetAsync(void* p, int v, size_t n, hipStream_t) { memset(p, v, n); return hipSuccess; }
inline hipError_t hipMemset(void* p, int v, size_t n) { memset(p, v, n); return hipSuccess; }
template <typename T>
inline hipError_t hipMalloc(T** p, size_t n) { *p = static_cast<T*>(calloc(1, n)); return *p ? hipSuccess : 1; }
inline hipError_t hipFree(void* p) { free(p); return hipSuccess; }
enum { hipMemcpyHostToDevice = 1, hipMemcpyDeviceToDevice = 3 };
inline hipError_t hipMemcpy(void* d, const void* s, size_t n, int) { memcpy(d, s, n); return hipSuccess; }
template <typename T>
inline hipError_t hipMemcpyFromSymbol(void* dst, T* sym, size_t n, size_t off, int) {
  memcpy(dst, (const char*)sym + off, n);
  return hipSuccess;
}

// ---- bit casts and correctly rounded arithmetic ----
inline uint32_t __float_as_uint(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float __uint_as_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
inline float __fdiv_rn(float a, float b) { return a / b; }
inline float __fmul_rn(float a, float b) { return a * b; }
inline float __fsub_rn(float a, float b) { return a - b; }
inline float __fadd_rn(float a, float b) { return a + b; }
inline unsigned long long __float2ull_rn(float f) { return (unsigned long long)std::nearbyint((double)f); }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }

// ---- atomics (global and "LDS" memory are host memory) ----
template <typename T> inline T atomicAdd(T* p, T v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline uint32_t atomicAdd(uint32_t* p, int v) { return __atomic_fetch_add(p, (uint32_t)v, __ATOMIC_SEQ_CST); }
template <typename T> inline T atomicOr(T* p, T v) { return __atomic_fetch_or(p, v, __ATOMIC_SEQ_CST); }
template <typename T> inline T atomicMin(T* p, T v) { return __atomic_fetch_min(p, v, __ATOMIC_SEQ_CST); }
template <typename T> inline T atomicMax(T* p, T v) { return __atomic_fetch_max(p, v, __ATOMIC_SEQ_CST); }
template <typename T> inline T atomicCAS(T* p, T cmp, T v) {
  __atomic_compare_exchange_n(p, &cmp, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);
  return cmp;
}
#define __HIP_MEMORY_SCOPE_AGENT 2
#define __HIP_MEMORY_SCOPE_WORKGROUP 1
#define __HIP_MEMORY_SCOPE_SYSTEM 3
#define __hip_atomic_load(p, order, scope) __atomic_load_n((p), (order))
#define __hip_atomic_store(p, v, order, scope) __atomic_store_n((p), (v), (order))
#define __hip_atomic_fetch_add(p, v, order, scope) __atomic_fetch_add((p), (v), (order))
#define __hip_atomic_exchange(p, v, order, scope) __atomic_exchange_n((p), (v), (order))

// ---- AMDGPU builtins ----
#define __builtin_amdgcn_fence(order, scope) __atomic_thread_fence(order)
#define __builtin_amdgcn_s_waitcnt(n) ((void)0)
#define __builtin_amdgcn_s_sleep(n) std::this_thread::yield()
#define __builtin_amdgcn_s_memrealtime() ((uint64_t)0)
// HW_REG_XCC_ID: the XCD a block id is dispatched to (round-robin over 8)
#define __builtin_amdgcn_s_getreg(reg) ((int)(::lps_emu::t_block.x & 7u))
#define __builtin_amdgcn_exp2f(x) exp2f(x)

inline uint64_t lps_emu_ballot(bool p) {
  return lps_emu::xchg<uint64_t>(p ? 1ull : 0ull, [](const uint64_t* b, uint64_t alive) {
    uint64_t m = 0;
    for (int l = 0; l < 64; l++)
      if (((alive >> l) & 1ull) && b[l]) m |= 1ull << l;
    return m;
  });
}
#define __builtin_amdgcn_ballot_w64(p) lps_emu_ballot((p))
#define __ballot(p) lps_emu_ballot((p))
inline bool __all(bool p) {
  return lps_emu::xchg<uint64_t>(p ? 1ull : 0ull, [](const uint64_t* b, uint64_t alive) -> uint64_t {
    for (int l = 0; l < 64; l++)
      if (((alive >> l) & 1ull) && !b[l]) return 0ull;
    return 1ull;
  }) != 0ull;
}
inline uint32_t __builtin_amdgcn_mbcnt_lo_emu(uint32_t m, uint32_t acc) {
  const int l = lps_emu::lane();
  const uint32_t below = l >= 32 ? 0xFFFFFFFFu : ((1u << l) - 1u);
  return acc + (uint32_t)__builtin_popcount(m & below);
}
inline uint32_t __builtin_amdgcn_mbcnt_hi_emu(uint32_t m, uint32_t acc) {
  const int l = lps_emu::lane();
  const uint32_t below = l < 32 ? 0u : ((1u << (l - 32)) - 1u);
  return acc + (uint32_t)__builtin_popcount(m & below);
}
#define __builtin_amdgcn_mbcnt_lo(m, a) __builtin_amdgcn_mbcnt_lo_emu((m), (a))
#define __builtin_amdgcn_mbcnt_hi(m, a) __builtin_amdgcn_mbcnt_hi_emu((m), (a))
inline int lps_emu_readlane(int v, int l) {
  return lps_emu::xchg<int>(v, [l](const uint64_t* b, uint64_t) { return (int)(uint32_t)b[l & 63]; });
}
inline int lps_emu_readfirstlane(int v) {
  return lps_emu::xchg<int>(v, [](const uint64_t* b, uint64_t alive) {
    return (int)(uint32_t)b[alive ? __builtin_ctzll(alive) : 0];
  });
}
#define __builtin_amdgcn_readlane(v, l) lps_emu_readlane((v), (l))
#define __builtin_amdgcn_readfirstlane(v) lps_emu_readfirstlane((v))
inline int lps_emu_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
  (void)bank_mask;
  const int me = lps_emu::lane();
  const int myold = old;
  return lps_emu::xchg<int>(src, [&](const uint64_t* b, uint64_t) {
    if (!((row_mask >> (me >> 4)) & 1)) return myold;
    const int s = lps_emu::dpp_src(me, ctrl);
    if (s < 0) return bound_ctrl ? 0 : myold;
    return (int)(uint32_t)b[s];
  });
}
#define __builtin_amdgcn_update_dpp(o, s, c, rm, bm, bc) lps_emu_dpp((o), (s), (c), (rm), (bm), (bc))

template <typename T>
inline T __shfl_xor(T v, int m, int w = 64) {
  (void)w;
  const int me = lps_emu::lane();
  return lps_emu::xchg<T>(v, [&](const uint64_t* b, uint64_t) { return lps_emu::from_bits<T>(b[(me ^ m) & 63]); });
}
template <typename T>
inline T __shfl_up(T v, unsigned d, int w = 64) {
  (void)w;
  const int me = lps_emu::lane();
  return lps_emu::xchg<T>(v, [&](const uint64_t* b, uint64_t) {
    return lps_emu::from_bits<T>(b[me >= (int)d ? me - (int)d : me]);
  });
}
template <typename T>
inline T __shfl(T v, int src, int w = 64) {
  (void)w;
  return lps_emu::xchg<T>(v, [&](const uint64_t* b, uint64_t) { return lps_emu::from_bits<T>(b[src & 63]); });
}

// Matrix-core instructions are not emulated (the LM-head kernel is not run here).
template <typename A, typename C>
inline C lps_emu_no_mfma(A, A, C c) {
  fprintf(stderr, "hostemu: matrix-core instructions are not emulated\n");
  abort();
  return c;
}
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, x, y, z) lps_emu_no_mfma((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, x, y, z) lps_emu_no_mfma((a), (b), (c))
