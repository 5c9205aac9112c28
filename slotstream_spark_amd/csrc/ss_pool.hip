// Expert slot pool in HBM with the reference's table ABI, CLOCK victim selection, generation pins and a
// transactional ensure that reads missing records from experts.bin (slotio/include/slotio/pool.hpp:39-165,
// slotio/src/clock.cpp, slotio/src/ensure.cpp; the file layout of docs/model-and-repack.md:37-57: the record of
// layer L, expert e at (L * E + e) * record_bytes).
//
// The reference keeps slots in host memory and streams records from NVMe; on MI355X the slots are HBM (288 GB
// holds every expert of the model), so the pool is a set of device chunks of `stride`-byte slots (the record rounded
// up to 256 bytes). The kernels read the two tables the caller owns in device memory: map int32 [layers * E]
// (expert of a layer -> slot, -1 = not resident) and slot_ptr int64 [max_slots] (slot -> record address). The misses
// of a call are spread over reader lanes (slotio's Reader has up to 12, reader.hpp:1): each lane preads a record into
// one of its two pinned staging buffers while the other one's copy to its slot runs on the lane's stream, so file
// reads, host-to-device copies and the lanes overlap. With `direct` the file is read with O_DIRECT (records and
// their offsets are then multiples of 4096 bytes; the page cache is bypassed as slotio's File::open_direct does).
// The table entries change only after every read of the call succeeded, and each phase (unmap, publish) updates
// the device map with one copy of the range it touched.
//
// Pins (a generation per slot, Pins::pin / retire_below) protect slots that in-flight work may still read: ensure
// pins every slot it returns with the caller's generation, and a slot becomes evictable again once the caller
// reports progress past that generation. Calls on one pool are serialised by its mutex.
#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "ss_launch.hpp"

namespace ss {

namespace {

int64_t now_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

}  // namespace

constexpr int kMaxLanes = 12;

struct Lane {
  void* staging[2] = {nullptr, nullptr};
  void* bounce = nullptr;  // 4096-aligned plain host memory for O_DIRECT reads (not into the pinned staging)
  hipEvent_t copied[2] = {nullptr, nullptr};
  hipStream_t stream = nullptr;
};

struct Pool {
  int layers = 0, experts = 0, max_slots = 0, slots = 0, slots_per_chunk = 0;
  int64_t record_bytes = 0, stride = 0, chunk_bytes = 0, file_bytes = 0;
  int fd = -1;         // buffered reads
  int fd_direct = -1;  // O_DIRECT reads when enabled
  std::string path;
  bool direct = false;
  int n_lanes = 1;
  int device = 0;  // the device current at open: slots, tables, streams and every lane thread use it
  std::vector<Lane> lanes;
  std::vector<void*> chunk_dev;
  int32_t* map_dev = nullptr;    // caller's device table [layers * experts]
  int64_t* ptr_dev = nullptr;    // caller's device table [max_slots]
  std::vector<int32_t> map;      // host mirror of map_dev
  std::vector<int64_t> slot_ptr; // host mirror of ptr_dev
  std::vector<int32_t> owner;    // slot -> layer * experts + e, or -1
  std::vector<uint8_t> ref;      // CLOCK reference bits
  int hand = 0;
  std::vector<int64_t> pin_gen;  // -1 = not pinned
  int pin_count = 0;
  const uint64_t* progress = nullptr;  // caller's progress word (host memory a kernel may advance), or null
  std::mutex mu;
  PoolStats st{};

  uint8_t* slot_dev(int s) const {
    return static_cast<uint8_t*>(chunk_dev[s / slots_per_chunk]) + (int64_t)(s % slots_per_chunk) * stride;
  }
  void pin(int s, int64_t gen) {
    if (pin_gen[s] < 0) ++pin_count;
    pin_gen[s] = std::max(pin_gen[s], gen);
  }
  bool pinned(int s) const { return pin_gen[s] >= 0; }
  // CLOCK: a global hand over the slots with reference bits; pinned slots are skipped. Fails after 3 * slots steps.
  int victim() {
    const long limit = 3L * slots;
    for (long i = 0; i < limit && slots > 0; ++i) {
      const int s = hand;
      hand = (hand + 1) % slots;
      if (pinned(s)) continue;
      if (ref[s]) {
        ref[s] = 0;
        continue;
      }
      return s;
    }
    return -1;
  }
  // One copy of map[lo, hi) to the device table (no-op for an empty range).
  hipError_t put_map(int64_t lo, int64_t hi) {
    if (hi <= lo) return hipSuccess;
    return hipMemcpy(map_dev + lo, &map[lo], (size_t)(hi - lo) * 4, hipMemcpyHostToDevice);
  }
  void drop_pins_below(uint64_t progress) {
    if (pin_count == 0) return;
    for (int s = 0; s < slots; ++s)
      if (pin_gen[s] >= 0 && (uint64_t)pin_gen[s] < progress) {
        pin_gen[s] = -1;
        --pin_count;
      }
  }
};

namespace {

hipError_t add_lanes(Pool* p, int n) {
  while ((int)p->lanes.size() < n) {
    p->lanes.emplace_back();
    Lane& ln = p->lanes.back();
    hipError_t e = hipStreamCreateWithFlags(&ln.stream, hipStreamNonBlocking);
    for (int k = 0; k < 2 && e == hipSuccess; ++k) {
      // 4096-aligned (hipHostMalloc returns page-aligned memory), as O_DIRECT reads need
      e = hipHostMalloc(&ln.staging[k], (size_t)p->record_bytes, hipHostMallocDefault);
      if (e == hipSuccess) e = hipEventCreateWithFlags(&ln.copied[k], hipEventDisableTiming);
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

void free_lane(Lane& ln) {
  if (ln.stream) (void)hipStreamSynchronize(ln.stream);
  free(ln.bounce);
  for (int k = 0; k < 2; ++k) {
    if (ln.staging[k]) (void)hipHostFree(ln.staging[k]);
    if (ln.copied[k]) (void)hipEventDestroy(ln.copied[k]);
  }
  if (ln.stream) (void)hipStreamDestroy(ln.stream);
}

// One lane's share of the misses (every `step`-th one from `first`): pread into the free staging buffer (O_DIRECT:
// into the lane's aligned bounce buffer, then a memcpy to staging, since direct I/O does not target the driver's
// pinned mappings), copy it to the victim slot on the lane's stream. Clears `ok` and records errno on a short read
// or a HIP error; the other lanes stop at their next record. Waits for the lane's copies before returning.
void read_lane(Pool* p, Lane& ln, const std::vector<int64_t>& offs, const std::vector<int32_t>& victims, size_t first,
               size_t step, std::atomic<bool>& ok, std::atomic<int64_t>& read_ns, std::atomic<int>& read_errno) {
  if (hipSetDevice(p->device) != hipSuccess) {  // a new thread starts on device 0
    ok = false;
    return;
  }
  const int fd = p->direct ? p->fd_direct : p->fd;
  int used = 0;
  for (size_t k = first; k < offs.size() && ok.load(std::memory_order_relaxed); k += step, ++used) {
    const int b = used & 1;
    if (used >= 2 && hipEventSynchronize(ln.copied[b]) != hipSuccess) {
      ok = false;
      break;
    }
    const int64_t r0 = now_ns();
    uint8_t* dst = static_cast<uint8_t*>(p->direct ? ln.bounce : ln.staging[b]);
    int64_t got = 0;
    while (got < p->record_bytes) {
      const ssize_t r = pread(fd, dst + got, (size_t)(p->record_bytes - got), (off_t)(offs[k] + got));
      if (r < 0) read_errno = errno;
      if (r <= 0) break;
      got += r;
    }
    if (p->direct && got == p->record_bytes) memcpy(ln.staging[b], ln.bounce, (size_t)p->record_bytes);
    read_ns += now_ns() - r0;
    if (got < p->record_bytes ||
        hipMemcpyAsync(p->slot_dev(victims[k]), ln.staging[b], (size_t)p->record_bytes, hipMemcpyHostToDevice,
                       ln.stream) != hipSuccess ||
        hipEventRecord(ln.copied[b], ln.stream) != hipSuccess) {
      ok = false;
      break;
    }
  }
  if (hipStreamSynchronize(ln.stream) != hipSuccess) ok = false;
}

}  // namespace

hipError_t pool_open(const char* path, int layers, int experts, int64_t record_bytes, int max_slots,
                     int64_t chunk_bytes, int32_t* map_dev, int64_t* ptr_dev, Pool** out, std::string* err) {
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    *err = std::string("cannot open ") + path;
    return hipErrorFileNotFound;
  }
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    ::close(fd);
    *err = std::string("cannot stat ") + path;
    return hipErrorFileNotFound;
  }
  Pool* p = new Pool();
  p->fd = fd;
  p->path = path;
  if (hipGetDevice(&p->device) != hipSuccess) p->device = 0;
  p->file_bytes = sb.st_size;
  p->layers = layers;
  p->experts = experts;
  p->record_bytes = record_bytes;
  p->stride = (record_bytes + 255) / 256 * 256;
  p->max_slots = max_slots;
  p->chunk_bytes = chunk_bytes;
  p->slots_per_chunk = (int)std::max<int64_t>(1, chunk_bytes / p->stride);
  p->map_dev = map_dev;
  p->ptr_dev = ptr_dev;
  p->map.assign((size_t)layers * experts, -1);
  p->slot_ptr.assign(max_slots, 0);
  p->owner.assign(max_slots, -1);
  p->ref.assign(max_slots, 0);
  p->pin_gen.assign(max_slots, -1);
  hipError_t e = hipMemcpy(map_dev, p->map.data(), p->map.size() * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(ptr_dev, p->slot_ptr.data(), p->slot_ptr.size() * 8, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = add_lanes(p, 1);
  if (e != hipSuccess) {
    pool_close(p);
    *err = "pool set-up failed";
    return e;
  }
  *out = p;
  return hipSuccess;
}

void pool_close(Pool* p) {
  if (!p) return;
  for (Lane& ln : p->lanes) free_lane(ln);
  for (void* c : p->chunk_dev) (void)hipFree(c);
  if (p->fd >= 0) ::close(p->fd);
  if (p->fd_direct >= 0) ::close(p->fd_direct);
  delete p;
}

// Reader set-up (slotio Reader::Config lanes, File::open_direct): 1..12 lanes; direct needs records and their file
// offsets to be multiples of 4096 bytes and a file system that takes O_DIRECT.
hipError_t pool_set_reader(Pool* p, int lanes, bool direct, std::string* err) {
  std::lock_guard<std::mutex> g(p->mu);
  if (lanes < 1 || lanes > kMaxLanes) {
    *err = "lanes must be 1.." + std::to_string(kMaxLanes);
    return hipErrorInvalidValue;
  }
  if (direct && p->fd_direct < 0) {
    if (p->record_bytes % 4096 != 0) {
      *err = "O_DIRECT needs record_bytes to be a multiple of 4096";
      return hipErrorInvalidValue;
    }
    p->fd_direct = ::open(p->path.c_str(), O_RDONLY | O_CLOEXEC | O_DIRECT);
    if (p->fd_direct < 0) {
      *err = "cannot open " + p->path + " with O_DIRECT";
      return hipErrorFileNotFound;
    }
  }
  hipError_t e = add_lanes(p, lanes);
  if (e != hipSuccess) {
    *err = "lane set-up failed";
    return e;
  }
  if (direct)
    for (int l = 0; l < lanes; ++l)
      if (!p->lanes[l].bounce && posix_memalign(&p->lanes[l].bounce, 4096, (size_t)p->record_bytes) != 0) {
        p->lanes[l].bounce = nullptr;
        *err = "bounce buffer allocation failed";
        return hipErrorOutOfMemory;
      }
  p->n_lanes = lanes;
  p->direct = direct;
  return hipSuccess;
}

// Grow: allocate chunks, publish the new slots' addresses. Shrink: unmap every slot >= n, drop its pin and
// reference bit, free the chunks no slot uses (Pool::resize_slots, Clock::drop_above, Pins::drop_above).
hipError_t pool_resize(Pool* p, int n, std::string* err) {
  std::lock_guard<std::mutex> g(p->mu);
  if (n < 0 || n > p->max_slots) {
    *err = "slots out of range";
    return hipErrorInvalidValue;
  }
  const int need = (n + p->slots_per_chunk - 1) / p->slots_per_chunk;
  if (n >= p->slots) {
    for (int c = (int)p->chunk_dev.size(); c < need; ++c) {
      void* d = nullptr;
      hipError_t e = hipMalloc(&d, (size_t)p->slots_per_chunk * p->stride);
      if (e != hipSuccess) {
        *err = "chunk allocation failed";
        return e;
      }
      p->chunk_dev.push_back(d);
    }
    for (int s = p->slots; s < n; ++s) p->slot_ptr[s] = reinterpret_cast<int64_t>(p->slot_dev(s));
  } else {
    int64_t lo = INT64_MAX, hi = 0;
    for (int s = n; s < p->slots; ++s) {
      if (p->owner[s] >= 0) {
        p->map[p->owner[s]] = -1;
        lo = std::min<int64_t>(lo, p->owner[s]);
        hi = std::max<int64_t>(hi, p->owner[s] + 1);
        p->owner[s] = -1;
      }
      p->slot_ptr[s] = 0;
      p->ref[s] = 0;
      if (p->pin_gen[s] >= 0) {
        p->pin_gen[s] = -1;
        --p->pin_count;
      }
    }
    if (p->hand >= n) p->hand = 0;
    hipError_t e = p->put_map(lo, hi);
    if (e != hipSuccess) return e;
    while ((int)p->chunk_dev.size() > need) {
      hipError_t e = hipFree(p->chunk_dev.back());
      if (e != hipSuccess) return e;
      p->chunk_dev.pop_back();
    }
  }
  const int lo = std::min(n, p->slots), hi = std::max(n, p->slots);
  p->slots = n;
  if (hi > lo) {
    hipError_t e = hipMemcpy(p->ptr_dev + lo, p->slot_ptr.data() + lo, (size_t)(hi - lo) * 8, hipMemcpyHostToDevice);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

void pool_retire_below(Pool* p, uint64_t progress) {
  std::lock_guard<std::mutex> g(p->mu);
  p->drop_pins_below(progress);
}

// ensure (slotio/src/ensure.cpp): (1) validate and dedupe in first-seen order; (2) capacity check, no state change
// on failure; (3) pin the hits; (4) choose and pin every victim; (5) unmap each victim's old owner; (6, 7) read the
// misses into their victims; (8) on a read error restore the pins, leave the victims unmapped, publish nothing;
// (9) publish. Returns the slot of every requested expert in input order.
PoolStatus pool_ensure(Pool* p, int layer, const int32_t* experts, int n, uint64_t gen, int32_t* out,
                       EnsureTiming* t, std::string* err) {
  std::lock_guard<std::mutex> g(p->mu);
  const int64_t t0 = now_ns();
  if (layer < 0 || layer >= p->layers) {
    *err = "layer out of range";
    return PoolStatus::Invalid;
  }
  // Ensurer::ensure retires the pins below the progress word first
  if (p->progress) p->drop_pins_below(__atomic_load_n(p->progress, __ATOMIC_ACQUIRE));
  std::vector<int32_t> uniq;
  std::unordered_map<int32_t, int> pos;
  for (int i = 0; i < n; ++i) {
    const int32_t e = experts[i];
    if (e < 0 || e >= p->experts) {
      *err = "expert id out of range";
      return PoolStatus::Invalid;
    }
    if (pos.emplace(e, (int)uniq.size()).second) uniq.push_back(e);
  }
  std::vector<int32_t> slot(uniq.size(), -1);
  std::vector<int> miss;
  int unpinned_hits = 0;
  for (size_t i = 0; i < uniq.size(); ++i) {
    const int32_t s = p->map[(size_t)layer * p->experts + uniq[i]];
    if (s >= 0) {
      slot[i] = s;
      if (!p->pinned(s)) ++unpinned_hits;
    } else {
      miss.push_back((int)i);
    }
  }
  if ((long)miss.size() > (long)p->slots - p->pin_count - unpinned_hits) {
    *err = "ensure needs " + std::to_string(miss.size()) + " slots, " +
           std::to_string(p->slots - p->pin_count - unpinned_hits) + " unpinned";
    return PoolStatus::Exhausted;
  }
  const std::vector<int64_t> snap = p->pin_gen;
  const int snap_count = p->pin_count;
  auto restore = [&]() {
    p->pin_gen = snap;
    p->pin_count = snap_count;
  };
  for (size_t i = 0; i < uniq.size(); ++i)
    if (slot[i] >= 0) {
      p->pin(slot[i], (int64_t)gen);
      p->ref[slot[i]] = 1;
    }
  std::vector<int32_t> victims;
  for (size_t k = 0; k < miss.size(); ++k) {
    const int v = p->victim();
    if (v < 0) {
      restore();
      *err = "CLOCK found no victim (all slots pinned)";
      return PoolStatus::Exhausted;
    }
    p->pin(v, (int64_t)gen);
    victims.push_back(v);
  }
  int64_t lo = INT64_MAX, hi = 0;
  for (int32_t v : victims) {
    if (p->owner[v] >= 0) {
      p->map[p->owner[v]] = -1;
      lo = std::min<int64_t>(lo, p->owner[v]);
      hi = std::max<int64_t>(hi, p->owner[v] + 1);
      p->owner[v] = -1;
    }
    p->ref[v] = 0;
  }
  if (p->put_map(lo, hi) != hipSuccess) {  // victims leave the table before their slots are overwritten
    restore();
    *err = "map update failed";
    return PoolStatus::Io;
  }
  const int64_t t_read = now_ns();
  std::vector<int64_t> offs(miss.size());
  for (size_t k = 0; k < miss.size(); ++k) offs[k] = ((int64_t)layer * p->experts + uniq[miss[k]]) * p->record_bytes;
  std::atomic<bool> ok{true};
  std::atomic<int64_t> read_ns{0};
  std::atomic<int> read_errno{0};
  const size_t nl = std::min<size_t>((size_t)p->n_lanes, miss.size());
  if (nl > 1) {
    std::vector<std::thread> th;
    for (size_t l = 1; l < nl; ++l)
      th.emplace_back(read_lane, p, std::ref(p->lanes[l]), std::cref(offs), std::cref(victims), l, nl, std::ref(ok),
                      std::ref(read_ns), std::ref(read_errno));
    read_lane(p, p->lanes[0], offs, victims, 0, nl, ok, read_ns, read_errno);
    for (auto& t : th) t.join();
  } else if (nl == 1) {
    read_lane(p, p->lanes[0], offs, victims, 0, 1, ok, read_ns, read_errno);
  }
  const int64_t t_copied = now_ns();
  if (!ok) {
    restore();
    *err = "ensure read failed (layer " + std::to_string(layer) + ")";
    if (read_errno.load()) *err += std::string(": ") + strerror(read_errno.load());
    return PoolStatus::Io;
  }
  lo = INT64_MAX;
  hi = 0;
  for (size_t k = 0; k < miss.size(); ++k) {
    const int32_t idx = layer * p->experts + uniq[miss[k]];
    p->owner[victims[k]] = idx;
    p->map[idx] = victims[k];
    lo = std::min<int64_t>(lo, idx);
    hi = std::max<int64_t>(hi, idx + 1);
    p->ref[victims[k]] = 1;
    slot[miss[k]] = victims[k];
  }
  if (p->put_map(lo, hi) != hipSuccess) {
    *err = "map update failed";
    return PoolStatus::Io;
  }
  for (int i = 0; i < n; ++i) out[i] = slot[pos[experts[i]]];
  p->st.hits += (int64_t)(uniq.size() - miss.size());
  p->st.misses += (int64_t)miss.size();
  p->st.bytes += (int64_t)miss.size() * p->record_bytes;
  if (t) {
    t->hits = (int64_t)(uniq.size() - miss.size());
    t->misses = (int64_t)miss.size();
    t->bytes = (int64_t)miss.size() * p->record_bytes;
    t->total_ns = now_ns() - t0;
    t->read_ns = read_ns.load() / (int64_t)std::max<size_t>(nl, 1);  // mean over the lanes
    t->copy_ns = std::max<int64_t>(0, t_copied - t_read - t->read_ns);
  }
  return PoolStatus::Ok;
}

void pool_set_progress(Pool* p, const uint64_t* progress) {
  std::lock_guard<std::mutex> g(p->mu);
  p->progress = progress;
}

hipError_t pool_copy_slot(Pool* p, int slot, void* dst, int64_t bytes, std::string* err) {
  std::lock_guard<std::mutex> g(p->mu);
  if (slot < 0 || slot >= p->slots || bytes < 0 || bytes > p->stride) {
    *err = "slot or size out of range";
    return hipErrorInvalidValue;
  }
  return hipMemcpy(dst, p->slot_dev(slot), (size_t)bytes, hipMemcpyDefault);
}

void pool_info(Pool* p, PoolStats* s) {
  std::lock_guard<std::mutex> g(p->mu);
  *s = p->st;
  s->slots = p->slots;
  s->chunks = (int64_t)p->chunk_dev.size();
  s->pinned = p->pin_count;
  s->owned_bytes = (int64_t)p->chunk_dev.size() * p->slots_per_chunk * p->stride;
  s->stride = p->stride;
  s->lanes = p->n_lanes;
  s->direct = p->direct ? 1 : 0;
}

}  // namespace ss
