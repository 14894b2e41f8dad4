// launchers.cpp -- the reference-named C++ launchers, forwarding to the C ABI.
//
// The reference's launchers return void and never check for errors; these
// keep the void signatures but throw std::runtime_error when the library
// rejects a launch, so a bad shape or a failed launch cannot pass silently.
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>

#include "kernels/gelu_kernel.h"
#include "kernels/model_utils_kernel.h"
#include "kernels/rmsnorm_kernel.h"
#include "kernels/rope_kernel.h"
#include "kernels/sampling_kernel.h"
#include "kernels/softmax_kernel.h"
#include "kernels/swiglu_kernel.h"
#include "mi_kernels.h"

namespace mini_infer {
namespace kernels {
namespace {

void check(int status, const char* what) {
    if (status != MI_OK)
        throw std::runtime_error(std::string(what) + ": " + mi_status_string(status));
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void* sv(hipStream_t s) { return reinterpret_cast<void*>(s); }

// Host positions reach the table kernel through pinned staging buffers the
// library holds: a ring of kSlots per device, each guarded by an event.  A
// call copies the caller's positions into a slot on the host, so the
// caller's buffer is free on return, and the table kernel reads them from the
// pinned slot directly (no device copy, no host wait); the slot's event,
// recorded after the kernel, keeps a later call from overwriting it early.
// The host waits only when a slot's previous kernel is still running.  Slots
// grow to the largest call seen and are kept until the process ends.
class PositionStager {
  public:
    static PositionStager& for_current_device() {
        static std::mutex mu;
        static std::map<int, PositionStager*> stagers;
        int dev = 0;
        hip_check(hipGetDevice(&dev), "launch_rope_precompute: hipGetDevice");
        std::lock_guard<std::mutex> lock(mu);
        PositionStager*& p = stagers[dev];
        if (!p) p = new PositionStager();
        return *p;
    }

    // Copies n positions into the next free slot and runs `use` with it
    // (device-readable pinned memory); then records the slot's event on s.
    template <typename Use>
    void run(const int64_t* src, int64_t n, hipStream_t s, Use use) {
        std::lock_guard<std::mutex> lock(mu_);
        Slot& slot = slots_[next_];
        next_ = (next_ + 1) % kSlots;
        if (slot.pending)
            hip_check(hipEventSynchronize(slot.ev), "launch_rope_precompute: slot wait");
        slot.pending = false;
        const size_t bytes = static_cast<size_t>(n) * sizeof(int64_t);
        if (slot.cap < bytes) {
            if (slot.host) hip_check(hipHostFree(slot.host), "launch_rope_precompute: hipHostFree");
            slot.host = nullptr;
            slot.cap = 0;
            const size_t cap = bytes < 4096 ? 4096 : bytes;
            hip_check(hipHostMalloc(reinterpret_cast<void**>(&slot.host), cap,
                                    hipHostMallocDefault),
                      "launch_rope_precompute: hipHostMalloc");
            slot.cap = cap;
        }
        if (!slot.ev)
            hip_check(hipEventCreateWithFlags(&slot.ev, hipEventDisableTiming),
                      "launch_rope_precompute: hipEventCreate");
        std::memcpy(slot.host, src, bytes);
        use(static_cast<const int64_t*>(slot.host));
        hip_check(hipEventRecord(slot.ev, s), "launch_rope_precompute: hipEventRecord");
        slot.pending = true;
    }

  private:
    static constexpr int kSlots = 4;
    struct Slot {
        int64_t* host = nullptr;
        size_t cap = 0;
        hipEvent_t ev = nullptr;
        bool pending = false;
    };
    std::mutex mu_;
    Slot slots_[kSlots];
    int next_ = 0;
};

}  // namespace

void launch_rmsnorm(const __half* x, const __half* weight, __half* y, int N, int D, float eps,
                    int add_one, hipStream_t stream) {
    check(mi_rmsnorm_f16(x, weight, y, N, D, eps, add_one, sv(stream)), "launch_rmsnorm");
}

void launch_fused_add_rmsnorm(const __half* x, __half* residual, const __half* weight, __half* y,
                              int N, int D, float eps, int add_one, hipStream_t stream) {
    check(mi_fused_add_rmsnorm_f16(x, residual, weight, y, N, D, eps, add_one, sv(stream)),
          "launch_fused_add_rmsnorm");
}

void launch_qk_rmsnorm(__half* q, __half* k, const __half* q_weight, const __half* k_weight,
                       int T, int Hq, int Hkv, int head_dim, float eps, int add_one,
                       hipStream_t stream) {
    check(mi_qk_rmsnorm_f16(q, k, q_weight, k_weight, T, Hq, Hkv, head_dim, eps, add_one,
                            sv(stream)),
          "launch_qk_rmsnorm");
}

void launch_rope(const __half* x, const __half* cos_t, const __half* sin_t, __half* y, int B,
                 int S, int H, int D, hipStream_t stream) {
    check(mi_rope_neox_f16(x, cos_t, sin_t, y, B, S, H, D, sv(stream)), "launch_rope");
}

void launch_rope_precompute_batched(const float* inv_freq_h, const int64_t* positions_h,
                                    __half* cos_d, __half* sin_d, int B, int S, int half,
                                    hipStream_t stream) {
    // The reference takes host positions (src/kernels/rope_kernel.cu:87-102
    // copies them with a per-call cudaMalloc and a synchronous copy).  Here
    // the table kernel reads them from the pinned staging ring: no device
    // allocation, copy or host wait (inv_freq travels by value in the kernel
    // arguments).
    const int64_t n = static_cast<int64_t>(B) * S;
    if (n <= 0 || half <= 0) return;
    if (!positions_h) throw std::runtime_error("launch_rope_precompute: null positions");
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hip_check(hipStreamIsCapturing(stream, &cap), "launch_rope_precompute: hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone)
        throw std::runtime_error(
            "launch_rope_precompute: host positions cannot be captured in a graph (a replay "
            "would re-read a reused staging buffer); use launch_rope_qk with device positions");
    int st = MI_OK;
    PositionStager::for_current_device().run(positions_h, n, stream, [&](const int64_t* pos) {
        st = mi_rope_tables_f16(inv_freq_h, pos, cos_d, sin_d, n, half, sv(stream));
    });
    check(st, "launch_rope_precompute");
}

void launch_rope_precompute(const float* inv_freq_h, const int64_t* positions_h, __half* cos_d,
                            __half* sin_d, int S, int half, hipStream_t stream) {
    launch_rope_precompute_batched(inv_freq_h, positions_h, cos_d, sin_d, 1, S, half, stream);
}

void launch_rope_qk(__half* q, __half* k, const int64_t* positions_d, const float* inv_freq_h,
                    int T, int Hq, int Hkv, int head_dim, hipStream_t stream) {
    check(mi_rope_neox_qk_f16(q, k, positions_d, inv_freq_h, T, Hq, Hkv, head_dim, sv(stream)),
          "launch_rope_qk");
}

void launch_bias_rope_qk(__half* q, __half* k, const __half* q_bias, const __half* k_bias,
                         const int64_t* positions_d, const float* inv_freq_h, int T, int Hq,
                         int Hkv, int head_dim, hipStream_t stream) {
    check(mi_bias_rope_neox_qk_f16(q, k, q_bias, k_bias, positions_d, inv_freq_h, T, Hq, Hkv,
                                   head_dim, sv(stream)),
          "launch_bias_rope_qk");
}

void launch_rope_kv_scatter(__half* q, __half* k, const __half* v, const __half* q_bias,
                            const __half* k_bias, const __half* v_bias,
                            const int64_t* positions_d, const float* inv_freq_h, int B, int S,
                            int Hq, int Hkv, int head_dim, __half* k_cache, __half* v_cache,
                            const int* block_table, const int* seq_len, const int* start_pos,
                            int layer, int num_blocks, int block_size, int max_blocks_per_seq,
                            hipStream_t stream) {
    const mi_kv_segment seg{0, B, S, block_table, seq_len, start_pos, max_blocks_per_seq};
    const int64_t T = static_cast<int64_t>(B) * S;
    const int st = mi_rope_kv_scatter_f16(q, k, v, q_bias, k_bias, v_bias, positions_d,
                                          inv_freq_h, T, Hq, Hkv, head_dim, k_cache, v_cache,
                                          layer, num_blocks, block_size, &seg, T > 0 ? 1 : 0,
                                          sv(stream));
    if (st != MI_ERR_UNSUPPORTED) {
        check(st, "launch_rope_kv_scatter");
        return;
    }
    if (q_bias)
        launch_bias_rope_qk(q, k, q_bias, k_bias, positions_d, inv_freq_h, B * S, Hq, Hkv,
                            head_dim, stream);
    else
        launch_rope_qk(q, k, positions_d, inv_freq_h, B * S, Hq, Hkv, head_dim, stream);
    launch_paged_kv_scatter_kv_bias(k, v, k_cache, v_cache, nullptr, v_bias, block_table, seq_len,
                                    start_pos, B, S, layer, num_blocks, Hkv, head_dim, block_size,
                                    max_blocks_per_seq, stream);
}

void launch_qk_norm_rope_kv_scatter(__half* q, __half* k, const __half* v,
                                    const __half* q_weight, const __half* k_weight,
                                    const int64_t* positions_d, const float* inv_freq_h, int B,
                                    int S, int Hq, int Hkv, int head_dim, float eps, int add_one,
                                    __half* k_cache, __half* v_cache, const int* block_table,
                                    const int* seq_len, const int* start_pos, int layer,
                                    int num_blocks, int block_size, int max_blocks_per_seq,
                                    hipStream_t stream) {
    const mi_kv_segment seg{0, B, S, block_table, seq_len, start_pos, max_blocks_per_seq};
    const int64_t T = static_cast<int64_t>(B) * S;
    const int st = mi_qk_norm_rope_kv_scatter_f16(
        q, k, v, q_weight, k_weight, positions_d, inv_freq_h, T, Hq, Hkv, head_dim, eps, add_one,
        k_cache, v_cache, layer, num_blocks, block_size, &seg, T > 0 ? 1 : 0, sv(stream));
    if (st != MI_ERR_UNSUPPORTED) {
        check(st, "launch_qk_norm_rope_kv_scatter");
        return;
    }
    launch_qk_norm_rope(q, k, q_weight, k_weight, positions_d, inv_freq_h, B * S, Hq, Hkv,
                        head_dim, eps, add_one, stream);
    launch_paged_kv_scatter_kv(k, v, k_cache, v_cache, block_table, seq_len, start_pos, B, S,
                               layer, num_blocks, Hkv, head_dim, block_size, max_blocks_per_seq,
                               stream);
}

void launch_qk_norm_rope(__half* q, __half* k, const __half* q_weight, const __half* k_weight,
                         const int64_t* positions_d, const float* inv_freq_h, int T, int Hq,
                         int Hkv, int head_dim, float eps, int add_one, hipStream_t stream) {
    check(mi_qk_norm_rope_f16(q, k, q_weight, k_weight, positions_d, inv_freq_h, T, Hq, Hkv,
                              head_dim, eps, add_one, sv(stream)),
          "launch_qk_norm_rope");
}

void launch_swiglu(const __half* gate, const __half* up, __half* out, int n, hipStream_t stream) {
    check(mi_swiglu_f16(gate, up, out, n, sv(stream)), "launch_swiglu");
}

void launch_gelu_tanh(const __half* x, __half* y, int64_t n, hipStream_t stream) {
    check(mi_gelu_tanh_f16(x, y, n, sv(stream)), "launch_gelu_tanh");
}

void launch_geglu(const __half* gate, const __half* up, __half* out, int64_t n,
                  hipStream_t stream) {
    check(mi_geglu_f16(gate, up, out, n, sv(stream)), "launch_geglu");
}

void launch_softmax(const __half* x, __half* y, int N, int D, hipStream_t stream) {
    check(mi_softmax_f16(x, y, N, D, sv(stream)), "launch_softmax");
}

void launch_add_bias(__half* y, const __half* bias, int M, int N, int batch_stride,
                     hipStream_t stream) {
    check(mi_add_bias_f16(y, bias, M, N, batch_stride, sv(stream)), "launch_add_bias");
}

void launch_add_inplace(__half* y, const __half* x, int64_t n, hipStream_t s) {
    check(mi_add_inplace_f16(y, x, n, sv(s)), "launch_add_inplace");
}

void launch_embedding_gather(const int64_t* token_ids, const __half* embed_table, __half* out,
                             int B, int S, int H, hipStream_t stream) {
    check(mi_embedding_gather_f16(token_ids, embed_table, out, static_cast<int64_t>(B) * S, H, 0,
                                  sv(stream)),
          "launch_embedding_gather");
}

void launch_scale_inplace(__half* y, float scale, int64_t n, hipStream_t stream) {
    check(mi_scale_inplace_f16(y, scale, n, sv(stream)), "launch_scale_inplace");
}

void launch_mul_inplace(__half* y, const __half* x, int64_t n, hipStream_t stream) {
    check(mi_mul_inplace_f16(y, x, n, sv(stream)), "launch_mul_inplace");
}

void launch_paged_kv_scatter(const __half* src, __half* cache, const int* block_table,
                             const int* seq_len, const int* start_pos, int B, int S, int layer,
                             int num_blocks, int H_kv, int D, int block_size,
                             int max_blocks_per_seq, hipStream_t stream) {
    check(mi_paged_kv_scatter_f16(src, cache, block_table, seq_len, start_pos, B, S, layer,
                                  num_blocks, H_kv, D, block_size, max_blocks_per_seq, sv(stream)),
          "launch_paged_kv_scatter");
}

void launch_paged_kv_scatter_kv(const __half* k_src, const __half* v_src, __half* k_cache,
                                __half* v_cache, const int* block_table, const int* seq_len,
                                const int* start_pos, int B, int S, int layer, int num_blocks,
                                int H_kv, int D, int block_size, int max_blocks_per_seq,
                                hipStream_t stream) {
    check(mi_paged_kv_scatter_kv_f16(k_src, v_src, k_cache, v_cache, block_table, seq_len,
                                     start_pos, B, S, layer, num_blocks, H_kv, D, block_size,
                                     max_blocks_per_seq, sv(stream)),
          "launch_paged_kv_scatter_kv");
}

void launch_paged_kv_scatter_kv_bias(const __half* k_src, const __half* v_src, __half* k_cache,
                                     __half* v_cache, const __half* k_bias, const __half* v_bias,
                                     const int* block_table, const int* seq_len,
                                     const int* start_pos, int B, int S, int layer,
                                     int num_blocks, int H_kv, int D, int block_size,
                                     int max_blocks_per_seq, hipStream_t stream) {
    check(mi_paged_kv_scatter_kv_bias_f16(k_src, v_src, k_cache, v_cache, k_bias, v_bias,
                                          block_table, seq_len, start_pos, B, S, layer,
                                          num_blocks, H_kv, D, block_size, max_blocks_per_seq,
                                          sv(stream)),
          "launch_paged_kv_scatter_kv_bias");
}

void launch_greedy_sample(const __half* logits, int vocab, int* out, hipStream_t stream) {
    check(mi_greedy_argmax_f16(logits, 1, vocab, out, sv(stream)), "launch_greedy_sample");
}

void launch_greedy_sample_batched(const __half* logits, int B, int vocab, int* out,
                                  hipStream_t stream) {
    if (B <= 0) return;
    check(mi_greedy_argmax_f16(logits, B, vocab, out, sv(stream)),
          "launch_greedy_sample_batched");
}

void launch_top_p_sample(const __half* logits, int vocab, float p, float temperature,
                         unsigned long long seed, int* out, hipStream_t stream) {
    check(mi_top_p_sample_f16(logits, vocab, p, temperature, seed, out, sv(stream)),
          "launch_top_p_sample");
}

void launch_top_p_sample_batched(const __half* logits, int B, int vocab, float p,
                                 float temperature, unsigned long long seed, int* out,
                                 hipStream_t stream) {
    if (B <= 0) return;
    check(mi_top_p_sample_batched_f16(logits, B, vocab, p, temperature, seed, out, sv(stream)),
          "launch_top_p_sample_batched");
}

}  // namespace kernels
}  // namespace mini_infer
