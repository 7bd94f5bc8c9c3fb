// Host worker threads of a context.  A proof runs its MSM jobs and the
// per-set window combinations of its three-set MSM on host threads; creating
// and joining a std::thread costs ~12 us on the GPU hosts, several times per
// proof, and a sleeping thread needs several microseconds to wake.  The
// workers here are started on first use and kept until the context is
// destroyed; while a proof runs (Hot) idle workers spin on the queue instead
// of sleeping, so a submitted task starts within a microsecond.
//
// Tasks must not throw.  finish() runs a task on the calling thread when no
// worker has taken it yet, so a caller never waits on a queued task: nested
// submissions (a job that splits its own work) cannot deadlock however many
// workers are busy.
#pragma once
#include <immintrin.h>

#include <atomic>
#include <condition_variable>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

namespace zk {

class WorkerPool {
 public:
  struct Task {
    std::function<void()> fn;
    std::atomic<int> state{0};  // 0 queued, 1 taken, 2 done
  };
  using TaskRef = std::shared_ptr<Task>;

  explicit WorkerPool(int workers) : want_(workers) {}
  WorkerPool(const WorkerPool&) = delete;
  WorkerPool& operator=(const WorkerPool&) = delete;
  ~WorkerPool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_.store(true, std::memory_order_release);
    }
    cv_.notify_all();
    for (std::thread& t : th_) t.join();
  }

  // Queues fn.  Returns nullptr, queuing nothing, when refuse is set or no
  // worker thread exists and none can be started; the caller then runs fn
  // itself.  Throws only what allocating the task throws.
  TaskRef submit(std::function<void()> fn, bool refuse = false) {
    if (refuse) return nullptr;
    TaskRef t = std::make_shared<Task>();
    t->fn = std::move(fn);
    {
      std::lock_guard<std::mutex> lk(mu_);
      while ((int)th_.size() < want_) {
        try {
          th_.emplace_back([this] { loop(); });
        } catch (...) {
          break;  // run with the workers there are
        }
      }
      if (th_.empty()) return nullptr;
      q_.push_back(t);
      pending_.fetch_add(1, std::memory_order_release);
    }
    cv_.notify_one();
    return t;
  }

  // Runs t here unless a worker has taken it; then waits until it is done.
  static void finish(const TaskRef& t) {
    if (!t) return;
    if (claim(*t)) {
      run(*t);
      return;
    }
    while (t->state.load(std::memory_order_acquire) != 2) _mm_pause();
  }

  // Idle workers spin instead of sleeping while at least one Hot lives.
  class Hot {
   public:
    explicit Hot(WorkerPool& p) : p_(p) {
      if (p_.hot_.fetch_add(1, std::memory_order_acq_rel) == 0) {
        // a worker tests hot_ under the mutex before it sleeps: taking the
        // mutex here orders this wake-up after that test
        { std::lock_guard<std::mutex> lk(p_.mu_); }
        p_.cv_.notify_all();
      }
    }
    ~Hot() { p_.hot_.fetch_sub(1, std::memory_order_acq_rel); }
    Hot(const Hot&) = delete;
    Hot& operator=(const Hot&) = delete;

   private:
    WorkerPool& p_;
  };

 private:
  static bool claim(Task& t) {
    int e = 0;
    return t.state.compare_exchange_strong(e, 1, std::memory_order_acq_rel);
  }
  static void run(Task& t) {
    t.fn();
    t.state.store(2, std::memory_order_release);
  }

  TaskRef pop() {
    if (pending_.load(std::memory_order_acquire) <= 0) return nullptr;
    std::lock_guard<std::mutex> lk(mu_);
    if (q_.empty()) return nullptr;
    TaskRef t = std::move(q_.front());
    q_.pop_front();
    pending_.fetch_sub(1, std::memory_order_release);
    return t;
  }

  void loop() {
    for (;;) {
      if (TaskRef t = pop()) {
        if (claim(*t)) run(*t);
        continue;
      }
      if (hot_.load(std::memory_order_acquire) > 0) {
        if (stop_.load(std::memory_order_acquire)) return;
        for (int i = 0; i < 64 && pending_.load(std::memory_order_acquire) <= 0; i++) _mm_pause();
        continue;
      }
      std::unique_lock<std::mutex> lk(mu_);
      cv_.wait(lk, [this] {
        return stop_.load(std::memory_order_acquire) || !q_.empty() || hot_.load(std::memory_order_acquire) > 0;
      });
      if (stop_.load(std::memory_order_acquire) && q_.empty()) return;
    }
  }

  const int want_;
  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<TaskRef> q_;
  std::vector<std::thread> th_;
  std::atomic<int> pending_{0};
  std::atomic<int> hot_{0};
  std::atomic<bool> stop_{false};
};

}  // namespace zk
