// A process-wide set of host worker threads for the library's host copies (the restore's host
// gather, the delivery into a staging file, the store's commit). A call hands the set n shares
// of work and waits for them; the threads are started on first use and then kept, asleep between
// calls, so a call does not start and join threads of its own. The delivery hands over one batch
// of rows every 0.5 ms or so, where starting 16 threads costs about as much as the copy.
//
// One call at a time has the set; a call that finds it busy (another thread of the process is in
// a call) runs its shares on threads of its own instead, so callers never wait for each other.
// The set is never destroyed: its threads sleep until the process ends, and nothing in it runs
// at exit. A child made by fork() inherits the set without its threads, and perhaps with its
// lock held by a thread that is not there: a call in any process other than the one that made
// the set runs on threads of its own and never touches the set.
#pragma once

#include <unistd.h>

#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace evs {

class Workers {
 public:
  static constexpr int kMaxThreads = 32;

  static Workers& get() {
    static Workers* const set = new Workers();  // kept to the process's end, never destroyed
    return *set;
  }

  // fn(0) .. fn(n - 1), the caller taking shares too; returns when every share is done.
  void run(int n, const std::function<void(int)>& fn) {
    if (n <= 1) {
      if (n == 1) fn(0);
      return;
    }
    if (getpid() != owner_) {  // a forked child: the set's threads are the parent's
      run_on_own_threads(n, fn);
      return;
    }
    std::unique_lock<std::mutex> mine(call_, std::try_to_lock);
    if (!mine.owns_lock()) {
      run_on_own_threads(n, fn);
      return;
    }
    start(n - 1 < kMaxThreads ? n - 1 : kMaxThreads);
    {
      std::lock_guard<std::mutex> hold(m_);
      fn_ = &fn;
      shares_ = n;
      next_ = 0;
      running_ = 0;
    }
    wake_.notify_all();
    for (;;) {
      int i;
      {
        std::lock_guard<std::mutex> hold(m_);
        if (next_ >= shares_) break;
        i = next_++;
        ++running_;
      }
      fn(i);
      finish();
    }
    std::unique_lock<std::mutex> hold(m_);
    done_.wait(hold, [&] { return running_ == 0 && next_ >= shares_; });
    fn_ = nullptr;
  }

 private:
  Workers() : owner_(getpid()) {}

  static void run_on_own_threads(int n, const std::function<void(int)>& fn) {
    std::vector<std::thread> own;
    own.reserve(static_cast<size_t>(n - 1));
    for (int i = 1; i < n; i++) own.emplace_back(fn, i);
    fn(0);
    for (auto& t : own) t.join();
  }

  void start(int want) {  // called with call_ held: only one caller starts threads
    while (static_cast<int>(threads_.size()) < want) threads_.emplace_back(&Workers::loop, this);
  }

  void finish() {
    std::lock_guard<std::mutex> hold(m_);
    if (--running_ == 0 && next_ >= shares_) done_.notify_all();
  }

  void loop() {
    std::unique_lock<std::mutex> hold(m_);
    for (;;) {
      wake_.wait(hold, [&] { return fn_ != nullptr && next_ < shares_; });
      const int i = next_++;
      ++running_;
      const std::function<void(int)>* fn = fn_;
      hold.unlock();
      (*fn)(i);
      hold.lock();
      if (--running_ == 0 && next_ >= shares_) done_.notify_all();
    }
  }

  const pid_t owner_;  // the process whose threads the set holds
  std::mutex call_;  // held by the call that has the set
  std::mutex m_;     // guards everything below
  std::condition_variable wake_, done_;
  const std::function<void(int)>* fn_ = nullptr;
  int shares_ = 0;
  int next_ = 0;     // the next share not yet taken
  int running_ = 0;  // shares taken and not yet finished
  std::vector<std::thread> threads_;  // never joined: the set outlives every call
};

// fn(0) .. fn(n - 1) on the library's worker threads and the caller.
inline void parallel_for(int n, const std::function<void(int)>& fn) {
  Workers::get().run(n, fn);
}

}  // namespace evs
