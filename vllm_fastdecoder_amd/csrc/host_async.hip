// Host-core partials in the background: fd_host_decode_partial_start queues
// one fd_host_decode_partial call for a runner thread of the library and
// returns at once; fd_host_decode_wait blocks until that call is done.
//
// The reference runs its host-tier kernel inside the forward, synchronously,
// after staging q on the host (fastdecode/backend.py:343-351). The hybrid
// split step instead overlaps the host cores' share of the host tier with
// the GPU's launch: the caller queues the host share right after enqueueing
// the copy of q to the host (with a HIP event recorded behind that copy),
// then enqueues the GPU's work, and waits when it needs the host partial.
// The runner waits for the event on its own thread, so the share starts as
// soon as q is on the host, with no thread of the caller's (nor its
// interpreter lock) in between; calls run one at a time, in queue order, on
// the same worker pool as fd_host_decode_partial.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>

#include <unistd.h>

#include "fd_common.h"
#include "host_decode.h"

namespace fd {
namespace {

// One queued fd_host_decode_partial call.
struct HostCall {
  int64_t id;
  hipEvent_t ready;  // waited for before the call (NULL: none)
  const void* q;
  int64_t q_ss, q_sh;
  const void* k;
  const void* v;
  int64_t sb, sh, st, num_blocks;
  const int32_t* bt;
  int64_t bt_stride;
  int32_t bt_width;
  const int32_t* lens;
  int32_t n, H, KVH, D, BS;
  float scale;
  int32_t kv_dt;
  void* out;
  int64_t out_ss, out_sh;
  int32_t out_dt;
  float* lse;
  int64_t lse_sh;
  int32_t threads;
};

struct CallState {
  bool done = false;
  int rc = FD_OK;
  double seconds = 0.0;  // the call itself, after the event
  std::string msg;
};

// The queue, the calls' states and the runner thread of one process. A child
// forked from a process that used them gets its own (the parent's runner
// thread does not exist in the child); the parent's are left alone there.
class Runner {
 public:
  explicit Runner(pid_t p) : pid(p) {}
  const pid_t pid;

  int64_t submit(HostCall c) {
    std::lock_guard<std::mutex> lk(mu_);
    c.id = next_id_++;
    states_.emplace(c.id, CallState{});
    queue_.push_back(c);
    if (!started_) {
      std::thread([this] { loop(); }).detach();  // lives as long as the process
      started_ = true;
    }
    work_cv_.notify_one();
    return c.id;
  }

  int wait(int64_t id, double* seconds) {
    std::unique_lock<std::mutex> lk(mu_);
    auto it = states_.find(id);
    if (it == states_.end())
      return set_error(FD_ERR_INVALID, "fd_host_decode_wait: no pending call %lld",
                       (long long)id);
    // (another thread waiting for the same call may take its state first)
    done_cv_.wait(lk, [&] {
      it = states_.find(id);
      return it == states_.end() || it->second.done;
    });
    if (it == states_.end())
      return set_error(FD_ERR_INVALID, "fd_host_decode_wait: call %lld already waited for",
                       (long long)id);
    const CallState s = it->second;
    states_.erase(it);
    lk.unlock();
    if (seconds != nullptr) *seconds = s.seconds;
    if (s.rc != FD_OK) return set_error(s.rc, "%s", s.msg.c_str());
    return FD_OK;
  }

 private:
  void loop() {
    for (;;) {
      HostCall c;
      {
        std::unique_lock<std::mutex> lk(mu_);
        work_cv_.wait(lk, [&] { return !queue_.empty(); });
        c = queue_.front();
        queue_.pop_front();
      }
      CallState s;
      if (c.ready != nullptr) {
        const hipError_t e = hipEventSynchronize(c.ready);
        if (e != hipSuccess) {
          s.rc = hip_error(e, "fd_host_decode_partial_start: hipEventSynchronize");
          s.msg = fd_last_error();
        }
      }
      if (s.rc == FD_OK) {
        const auto t0 = std::chrono::steady_clock::now();
        s.rc = fd_host_decode_partial(c.q, c.q_ss, c.q_sh, c.k, c.v, c.sb, c.sh, c.st,
                                      c.num_blocks, c.bt, c.bt_stride, c.bt_width, c.lens, c.n,
                                      c.H, c.KVH, c.D, c.BS, c.scale, c.kv_dt, c.out, c.out_ss,
                                      c.out_sh, c.out_dt, c.lse, c.lse_sh, c.threads);
        s.seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        if (s.rc != FD_OK) s.msg = fd_last_error();
      }
      s.done = true;
      {
        std::lock_guard<std::mutex> lk(mu_);
        states_[c.id] = s;
      }
      done_cv_.notify_all();
    }
  }

  std::mutex mu_;
  std::condition_variable work_cv_, done_cv_;
  std::deque<HostCall> queue_;
  std::unordered_map<int64_t, CallState> states_;
  int64_t next_id_ = 1;
  bool started_ = false;
};

Runner& runner() {
  static std::atomic<Runner*> state{nullptr};
  static std::mutex create_mu;  // taken only to create the runner of a process
  const pid_t me = getpid();
  Runner* r = state.load(std::memory_order_acquire);
  if (r != nullptr && r->pid == me) return *r;
  std::lock_guard<std::mutex> lk(create_mu);
  r = state.load(std::memory_order_acquire);
  if (r == nullptr || r->pid != me) {
    r = new Runner(me);  // intentionally never freed (its thread runs until the process ends)
    state.store(r, std::memory_order_release);
  }
  return *r;
}

}  // namespace
}  // namespace fd

using namespace fd;

extern "C" {

int fd_host_decode_partial_start(
    void* ready_event, const void* q, int64_t q_stride_seq, int64_t q_stride_head,
    const void* k_cache, const void* v_cache, int64_t kv_stride_block, int64_t kv_stride_head,
    int64_t kv_stride_token, int64_t num_blocks, const int32_t* block_table, int64_t bt_stride,
    int32_t bt_width, const int32_t* lens, int32_t n, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_size, int32_t block_size, float scale, int32_t kv_dtype, void* out,
    int64_t out_stride_seq, int64_t out_stride_head, int32_t out_dtype, float* lse,
    int64_t lse_stride_head, int32_t num_threads, int64_t* call) {
  return guarded("fd_host_decode_partial_start", [&]() -> int {
    if (call == nullptr)
      return set_error(FD_ERR_INVALID, "fd_host_decode_partial_start: call is NULL");
    const int rc = host_decode_check(q, k_cache, v_cache, num_blocks, block_table, bt_stride,
                                     bt_width, lens, n, num_heads, num_kv_heads, head_size,
                                     block_size, scale, kv_dtype, out, out_dtype, lse, num_threads);
    if (rc != FD_OK) return rc;
    HostCall c{0, static_cast<hipEvent_t>(ready_event), q, q_stride_seq, q_stride_head, k_cache,
               v_cache, kv_stride_block, kv_stride_head, kv_stride_token, num_blocks, block_table,
               bt_stride, bt_width, lens, n, num_heads, num_kv_heads, head_size, block_size, scale,
               kv_dtype, out, out_stride_seq, out_stride_head, out_dtype, lse, lse_stride_head,
               num_threads};
    *call = runner().submit(c);
    return FD_OK;
  });
}

int fd_host_decode_wait(int64_t call, double* seconds) {
  return guarded("fd_host_decode_wait", [&]() -> int { return runner().wait(call, seconds); });
}

int fd_hybrid_share_start(
    void* stream, void* ready_event, const void* q, void* q_host, const int32_t* host_bt,
    int64_t bt_stride, int32_t bt_width, const int32_t* host_lens, double cpu_fraction,
    int32_t* gpu_lens, int32_t* cpu_bt, int64_t cpu_bt_stride, int32_t* cpu_lens,
    const void* k_cache, const void* v_cache, int64_t kv_stride_block, int64_t kv_stride_head,
    int64_t kv_stride_token, int64_t num_blocks, int32_t n, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_size, int32_t block_size, float scale, int32_t kv_dtype,
    float* out, float* lse, int32_t num_threads, int64_t* call) {
  return guarded("fd_hybrid_share_start", [&]() -> int {
    if (call == nullptr) return set_error(FD_ERR_INVALID, "fd_hybrid_share_start: call is NULL");
    *call = 0;
    // the host call's checks, on the buffers it will read and write
    int rc = host_decode_check(q_host, k_cache, v_cache, num_blocks, cpu_bt, cpu_bt_stride,
                               bt_width, cpu_lens, n, num_heads, num_kv_heads, head_size,
                               block_size, scale, kv_dtype, out, FD_F32, lse, num_threads);
    if (rc != FD_OK) return rc;
    if (!(cpu_fraction >= 0.0 && cpu_fraction <= 1.0))
      return set_error(FD_ERR_INVALID, "fd_hybrid_share_start: cpu_fraction must be in [0, 1]");
    if (n == 0) return FD_OK;
    if (q == nullptr || ready_event == nullptr || (bt_width > 0 && host_bt == nullptr) ||
        host_lens == nullptr || gpu_lens == nullptr)
      return set_error(FD_ERR_INVALID, "fd_hybrid_share_start: NULL pointer");
    if (bt_stride < bt_width || cpu_bt_stride < std::max<int32_t>(bt_width, 1))
      return set_error(FD_ERR_INVALID,
                       "fd_hybrid_share_start: a table's row stride is below its width");
    // q on its way to the host first: the copy overlaps the share below
    const size_t elt = kv_dtype == FD_F32 ? 4 : 2;
    const int64_t row = (int64_t)num_heads * head_size;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(q_host, q, (size_t)n * row * elt, hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return hip_error(e, "fd_hybrid_share_start: copy of q to the host");
    e = hipEventRecord(static_cast<hipEvent_t>(ready_event), s);
    if (e != hipSuccess) return hip_error(e, "fd_hybrid_share_start: hipEventRecord");
    int32_t width = 0;
    rc = fd_share_host_blocks(host_bt, bt_stride, bt_width, host_lens, n, block_size,
                              cpu_fraction, gpu_lens, cpu_bt, cpu_bt_stride, cpu_lens, &width);
    if (rc != FD_OK) return rc;
    HostCall c{0, static_cast<hipEvent_t>(ready_event), q_host, row, head_size, k_cache, v_cache,
               kv_stride_block, kv_stride_head, kv_stride_token, num_blocks, cpu_bt, cpu_bt_stride,
               std::max<int32_t>(width, 1), cpu_lens, n, num_heads, num_kv_heads, head_size,
               block_size, scale, kv_dtype, out, row, head_size, FD_F32, lse, n, num_threads};
    *call = runner().submit(c);
    return FD_OK;
  });
}

}  // extern "C"
