// CPU build of generated porch kernels — TEST INFRASTRUCTURE ONLY.
//
// Lets a generated HIP kernel source compile as host C++ (clang) and run
// with one std::thread per work-item, so that every memory access it makes
// can be checked on the CPU against the exact buffer sizes: the driver
// places each buffer against an inaccessible guard region, and an access
// outside a buffer faults in this process instead of on a GPU.  Values are
// not the point (the oracle checks those); addresses are.
//
// Emulated: thread/block indices, __syncthreads (a barrier over the
// block's threads), __builtin_amdgcn_wave_barrier (a barrier over the
// wave's threads: on the GPU a wave's lanes run together and only the
// compiler's ordering is at stake), wave64 __shfl_xor, __shfl, __ballot,
// DPP row patterns,
// v_mfma_f32_32x32x2f32 and v_mfma_f32_16x16x4f32 (barriers
// over the wave's 64 threads, operand layouts as on gfx950), raw buffer
// stores (range-checked against the resource's size), LDS arrays
// (function-local statics, shared by the block's threads; blocks run one
// after another), relaxed 64-bit atomic loads and stores (host atomics; a
// block that waits on another block's store sees it only if that block ran
// earlier, so the emulation caps such waits: emulate.py).  The rest of the
// device builtins map to host math.
#pragma once

#include <barrier>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <thread>

namespace emu {
    struct dim3 {
        unsigned x = 0, y = 0, z = 0;
    };
    inline thread_local dim3 thread_idx;
    inline thread_local dim3 block_idx;
    inline dim3 grid_dim;
    inline dim3 block_dim;
    inline std::barrier<>* block_barrier = nullptr;
    inline std::barrier<>* wave_barrier[16] = {};
    inline float wave_a[16][64];
    inline float wave_b[16][64];

    inline int wave() { return static_cast<int>(thread_idx.x / 64); }
    inline int lane() { return static_cast<int>(thread_idx.x % 64); }
    inline void syncthreads() { block_barrier->arrive_and_wait(); }
    inline void wave_sync() { wave_barrier[wave()]->arrive_and_wait(); }

    inline float shfl_xor(float v, int mask, int width) {
        const int w = wave();
        const int l = lane();
        wave_a[w][l] = v;
        wave_barrier[w]->arrive_and_wait();
        const int src = ((l ^ mask) & (width - 1)) | (l & ~(width - 1));
        const float r = wave_a[w][src];
        wave_barrier[w]->arrive_and_wait();
        return r;
    }

    inline float shfl(float v, int src_lane, int width) {
        const int w = wave();
        const int l = lane();
        wave_a[w][l] = v;
        wave_barrier[w]->arrive_and_wait();
        const int src = (src_lane & (width - 1)) | (l & ~(width - 1));
        const float r = wave_a[w][src];
        wave_barrier[w]->arrive_and_wait();
        return r;
    }

    inline unsigned long long ballot(bool p) {
        const int w = wave();
        const int l = lane();
        wave_a[w][l] = p ? 1.0f : 0.0f;
        wave_barrier[w]->arrive_and_wait();
        unsigned long long mask = 0;
        for (int i = 0; i < 64; ++i)
            if (wave_a[w][i] != 0.0f) mask |= 1ull << i;
        wave_barrier[w]->arrive_and_wait();
        return mask;
    }

    // DPP row patterns used by the kernels: quad_perm [1,0,3,2] and
    // [2,3,0,1], row_half_mirror, row_mirror.
    inline int update_dpp(int src, int ctrl) {
        const int w = wave();
        const int l = lane();
        int from = l;
        if (ctrl == 0xB1) from = l ^ 1;
        else if (ctrl == 0x4E) from = l ^ 2;
        else if (ctrl == 0x141) from = (l & ~7) | (7 - (l & 7));
        else if (ctrl == 0x140) from = (l & ~15) | (15 - (l & 15));
        else std::abort();
        wave_a[w][l] = __builtin_bit_cast(float, src);
        wave_barrier[w]->arrive_and_wait();
        const float r = wave_a[w][from];
        wave_barrier[w]->arrive_and_wait();
        return __builtin_bit_cast(int, r);
    }

    typedef float v16 __attribute__((ext_vector_type(16)));

    // v_mfma_f32_32x32x2f32: lane l holds A[l % 32][l / 32] and
    // B[l / 32][l % 32]; accumulator register v of lane l is
    // C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
    inline v16 mfma_32x32x2(float a, float b, v16 c) {
        const int w = wave();
        const int l = lane();
        wave_a[w][l] = a;
        wave_b[w][l] = b;
        wave_barrier[w]->arrive_and_wait();
        v16 out = c;
        for (int v = 0; v < 16; ++v) {
            const int i = 8 * (v / 4) + 4 * (l / 32) + v % 4;
            const int j = l % 32;
            out[v] = c[v] + wave_a[w][i] * wave_b[w][j] + wave_a[w][i + 32] * wave_b[w][j + 32];
        }
        wave_barrier[w]->arrive_and_wait();
        return out;
    }

    typedef float v4 __attribute__((ext_vector_type(4)));

    // v_mfma_f32_16x16x4f32: lane l holds A[l % 16][l / 16] and
    // B[l / 16][l % 16]; accumulator register v of lane l is
    // C[4 (l / 16) + v][l % 16].
    inline v4 mfma_16x16x4(float a, float b, v4 c) {
        const int w = wave();
        const int l = lane();
        wave_a[w][l] = a;
        wave_b[w][l] = b;
        wave_barrier[w]->arrive_and_wait();
        v4 out = c;
        for (int v = 0; v < 4; ++v) {
            const int i = 4 * (l / 16) + v;
            const int j = l % 16;
            float sum = 0.0f;
            for (int kk = 0; kk < 4; ++kk) sum += wave_a[w][16 * kk + i] * wave_b[w][16 * kk + j];
            out[v] = c[v] + sum;
        }
        wave_barrier[w]->arrive_and_wait();
        return out;
    }

    // A raw buffer resource (stride 0): stores at byte offsets at or past
    // num_records are dropped, as the hardware's range check does.
    struct buffer_rsrc {
        char* base;
        uint32_t num_records;
    };
    inline void buffer_store_b32(unsigned int value, buffer_rsrc r, int offset) {
        const uint32_t at = static_cast<uint32_t>(offset);
        if (at >= r.num_records) return;
        __builtin_memcpy(r.base + at, &value, 4);
    }
} // namespace emu

#define threadIdx (emu::thread_idx)
#define blockIdx (emu::block_idx)
#define gridDim (emu::grid_dim)
#define blockDim (emu::block_dim)
#define __global__
#define __device__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static
#define __restrict__ __restrict
#define __syncthreads() emu::syncthreads()
#define __shfl_xor(v, m, w) emu::shfl_xor((v), (m), (w))
#define __shfl(v, s, w) emu::shfl((v), (s), (w))
#define __ballot(p) emu::ballot(p)
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define __builtin_amdgcn_exp2f(x) exp2f(x)
#define __builtin_amdgcn_sched_group_barrier(a, b, c) ((void)0)
#define __builtin_amdgcn_sched_barrier(a) ((void)0)
#define __builtin_amdgcn_wave_barrier() emu::wave_sync()
// the kernels read only wave-uniform values through it
#define __builtin_amdgcn_readfirstlane(x) (x)
#define __builtin_amdgcn_s_sleep(n) std::this_thread::yield()
#define __HIP_MEMORY_SCOPE_AGENT 0
#define __hip_atomic_load(p, order, scope) __atomic_load_n((p), (order))
#define __hip_atomic_store(p, v, order, scope) __atomic_store_n((p), (v), (order))
#define __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, x, y, z) emu::mfma_32x32x2((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, x, y, z) emu::mfma_16x16x4((a), (b), (c))
#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc) emu::update_dpp((src), (ctrl))
#define __builtin_amdgcn_make_buffer_rsrc(p, stride, num, flags) \
    emu::buffer_rsrc{reinterpret_cast<char*>(p), static_cast<uint32_t>(num)}
#define __builtin_amdgcn_raw_buffer_store_b32(v, r, off, soff, aux) emu::buffer_store_b32((v), (r), (off) + (soff))

struct __attribute__((aligned(16))) float4 {
    float x, y, z, w;
};
struct __attribute__((aligned(8))) float2 {
    float x, y;
};
inline float4 make_float4(float a, float b, float c, float d) { return {a, b, c, d}; }
inline float2 make_float2(float a, float b) { return {a, b}; }
