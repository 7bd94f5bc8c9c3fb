// Stress program for cuda-zkml_amd/csrc/worker_pool.hpp (tests/test_worker_pool.py
// builds it, also under ThreadSanitizer): many small tasks, tasks that split
// themselves into sub-tasks (nested submit + finish) on pools smaller than the
// nesting needs, several submitting threads, refused submissions, and pools
// destroyed while their workers sleep or spin.  Exit code 0 when every task
// ran exactly once.
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>

#include "worker_pool.hpp"

using zk::WorkerPool;

static int check(bool ok, const char* what) {
  if (!ok) fprintf(stderr, "FAIL: %s\n", what);
  return ok ? 0 : 1;
}

int main() {
  int bad = 0;
  for (int workers : {1, 2, 5}) {
    for (int hot : {0, 1}) {
      WorkerPool pool(workers);
      std::unique_ptr<WorkerPool::Hot> h;
      if (hot) h.reset(new WorkerPool::Hot(pool));
      // flat: 2000 tasks, finished in submission order
      std::atomic<int> count{0};
      std::vector<WorkerPool::TaskRef> ts;
      for (int i = 0; i < 2000; i++) ts.push_back(pool.submit([&count] { count.fetch_add(1); }));
      for (auto& t : ts) WorkerPool::finish(t);
      bad += check(count.load() == 2000, "flat tasks ran once each");
      // nested: each of 50 tasks splits into 4 sub-tasks and waits for them
      std::atomic<int> leaves{0};
      std::vector<WorkerPool::TaskRef> outer;
      for (int i = 0; i < 50; i++)
        outer.push_back(pool.submit([&pool, &leaves] {
          std::vector<WorkerPool::TaskRef> in;
          for (int k = 0; k < 4; k++) in.push_back(pool.submit([&leaves] { leaves.fetch_add(1); }));
          for (auto& t : in) WorkerPool::finish(t);
        }));
      for (auto& t : outer) WorkerPool::finish(t);
      bad += check(leaves.load() == 200, "nested tasks ran once each");
      // several submitting threads
      std::atomic<int> multi{0};
      std::vector<std::thread> subs;
      for (int s = 0; s < 4; s++)
        subs.emplace_back([&pool, &multi] {
          std::vector<WorkerPool::TaskRef> mine;
          for (int i = 0; i < 300; i++) mine.push_back(pool.submit([&multi] { multi.fetch_add(1); }));
          for (auto& t : mine) WorkerPool::finish(t);
        });
      for (auto& t : subs) t.join();
      bad += check(multi.load() == 1200, "tasks of several submitters ran once each");
      // refused submission queues nothing; finish(nullptr) is a no-op
      bad += check(pool.submit([] {}, true) == nullptr, "refused submission returns null");
      WorkerPool::finish(nullptr);
      // a Hot guard that ends while workers spin, then the pool's destruction
      h.reset();
    }
  }
  if (!bad) printf("worker pool ok\n");
  return bad;
}
