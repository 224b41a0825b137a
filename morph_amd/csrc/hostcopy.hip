// Parallel host memory copy for the pinned staging of pageable host tensors.
//
// Host code only: no GPU work.  The staging copies each chunk of a pageable
// host tensor into a pinned buffer before its DMA (and out of one after a
// DMA back).  torch's copy_ runs those copies on its intra-op threads, one per
// core by default; measured on the MI355X box (16 cores), a staged round trip
// of the config-2 masters then took 6.3 to 133 ms from run to run (24 ms
// median), against a steady 6.7 ms with 12 threads: the copy threads that
// spin after each copy leave no core to the HIP runtime threads and the
// thread that queues the DMAs.  This pool copies with a thread count the
// caller chooses, and its workers sleep on a condition variable when idle:
// the streamed config-2 step went from 13.8-18.2 ms (torch, 16 threads) to
// 11.0-11.8 ms (8 threads here), config 5 from 155-163 ms to 139-140 ms.
//
// The calling thread copies pieces too, so every call completes even when no
// worker runs (a forked child gets a new pool: the parent's workers do not
// exist there).  Calls are serialized.  The pool is never destroyed: workers
// blocked on its condition variable at process exit must not see it torn down.
#include <unistd.h>

#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <system_error>
#include <thread>

#include "common.h"

namespace morph {
namespace {

constexpr int kMaxCopyThreads = 64;
// Pieces of at least 1 MiB: waking a sleeping worker costs more than copying
// a smaller piece on the calling thread.
constexpr size_t kMinPieceBytes = size_t(1) << 20;

struct CopyPool {
  std::mutex call;  // one copy at a time
  std::mutex m;
  std::condition_variable work, done;
  int workers = 0;
  pid_t pid = getpid();
  // the copy in progress
  char* dst = nullptr;
  const char* src = nullptr;
  size_t bytes = 0, piece = 0;
  int pieces = 0, next = 0, remaining = 0;

  // Take and copy pieces until none is left; `lk` holds m on entry and exit.
  void drain(std::unique_lock<std::mutex>& lk) {
    while (next < pieces) {
      const int i = next++;
      char* d = dst;
      const char* s = src;
      const size_t lo = (size_t)i * piece, n = lo + piece < bytes ? piece : bytes - lo;
      lk.unlock();
      std::memcpy(d + lo, s + lo, n);
      lk.lock();
      if (--remaining == 0) done.notify_all();
    }
  }

  void worker() {
    std::unique_lock<std::mutex> lk(m);
    for (;;) {
      work.wait(lk, [this] { return next < pieces; });
      drain(lk);
    }
  }

  void grow(int n) {
    std::lock_guard<std::mutex> lk(m);
    try {
      for (; workers < n; ++workers) std::thread([this] { worker(); }).detach();
    } catch (const std::system_error&) {
      // no more threads: the workers there are, and the caller, copy every piece
    }
  }
};

CopyPool* pool_for_this_process() {
  static std::mutex guard;
  static CopyPool* pool = nullptr;
  std::lock_guard<std::mutex> lk(guard);
  if (pool == nullptr || pool->pid != getpid()) pool = new CopyPool();  // the old one is left
  return pool;
}

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int morph_host_copy(void* dst, const void* src, size_t bytes, int threads) {
  if (bytes == 0) return MORPH_OK;
  if (dst == nullptr || src == nullptr || threads < 1) return MORPH_EINVAL;
  if (threads > kMaxCopyThreads) return MORPH_ERANGE;
  const uintptr_t d = reinterpret_cast<uintptr_t>(dst), s = reinterpret_cast<uintptr_t>(src);
  if (d < s + bytes && s < d + bytes) return MORPH_EINVAL;  // the ranges overlap
  size_t piece = (bytes + threads - 1) / threads;
  if (piece < kMinPieceBytes) piece = kMinPieceBytes;
  piece = (piece + 63) & ~size_t(63);
  const int pieces = (int)((bytes + piece - 1) / piece);
  if (pieces == 1) {
    std::memcpy(dst, src, bytes);
    return MORPH_OK;
  }
  CopyPool* p = pool_for_this_process();
  std::lock_guard<std::mutex> call(p->call);
  p->grow(pieces - 1);  // the caller takes pieces as well
  std::unique_lock<std::mutex> lk(p->m);
  p->dst = static_cast<char*>(dst);
  p->src = static_cast<const char*>(src);
  p->bytes = bytes;
  p->piece = piece;
  p->pieces = pieces;
  p->next = 0;
  p->remaining = pieces;
  p->work.notify_all();
  p->drain(lk);
  p->done.wait(lk, [p] { return p->remaining == 0; });
  p->pieces = 0;
  p->next = 0;
  return MORPH_OK;
}
