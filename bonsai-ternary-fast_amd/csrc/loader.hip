// loader.hip -- the load path's staged upload: PTQ1_0 rows from host memory
// (typically the GGUF mapping) into the resident T2 layout on the device,
// and the plan of the resident bytes (C ABI btf_hip_loader_* and
// btf_hip_gguf_plan).
//
// Behaviour of the reference's GpuDecoder::upload_mat / upload
// (src/cuda/gpu_decoder.cu:284-300, 302-393): a matrix is moved in slices of
// whole rows through two pinned staging slots in turn; before a slot is
// refilled the host waits for the event recorded after its previous slice's
// repack, so the host's copy of one slice overlaps the device's work on the
// other. The host copy of a slice runs on a pool of up to 16 threads started
// with the loader. The reference's
// repack kernel reads a mapped pinned slot across the bus; here each slice is
// instead copied by the DMA engine into a device staging slot
// (hipMemcpyAsync) and repacked from HBM, so the repack kernel never runs at
// bus speed and the copy engines carry the transfer. Results are
// byte-identical to repacking on the host (src/repack.cpp:16-27).
//
// The plan follows the packed-matrix items of the reference's plan_memory
// (src/repack.cpp:142-204): resident codes (K/4 B per row) and fp16 scales
// (K/64 B per row) of every PTQ1_0 matrix, and the staging, freed after the
// load. The rest of the reference's plan (KV cache, recurrent state,
// activations) belongs to the decoder, outside this path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/btf/hip_abi.h"
#include "common.h"

namespace btfhip {

// Worker threads for the host copy of a slice, started once with the loader:
// a slice is cut into parts of at least 1 MiB, part 0 copied by the calling
// thread and part t by worker t - 1 (one thread copies a page-cache mapping
// at ~10 GB/s; the copy engine moves ~55 GB/s).
struct CopyPool {
  std::vector<std::thread> workers;
  std::mutex mu;
  std::condition_variable go, done;
  uint64_t gen = 0;  // job number
  int pending = 0;   // workers still copying the current job
  bool stop = false;
  char* dst = nullptr;
  const char* src = nullptr;
  size_t bytes = 0, part = 0;
  int nparts = 0;

  void run(int t) {  // worker t copies part t + 1
    uint64_t seen = 0;
    for (;;) {
      std::unique_lock<std::mutex> lk(mu);
      go.wait(lk, [&] { return stop || gen != seen; });
      if (stop) return;
      seen = gen;
      const int k = t + 1;
      const bool mine = k < nparts;
      char* d = dst;
      const char* sp = src;
      const size_t b = std::min(bytes, (size_t)k * part), e = std::min(bytes, (size_t)(k + 1) * part);
      lk.unlock();
      if (mine && e > b) std::memcpy(d + b, sp + b, e - b);
      lk.lock();
      if (--pending == 0) done.notify_one();
    }
  }
  void start(int n) {  // fewer workers if the system refuses threads
    try {
      for (int t = 0; t < n; ++t) workers.emplace_back([this, t] { run(t); });
    } catch (const std::exception&) {
    }
  }
  void copy(void* d, const void* sp, size_t n_bytes) {
    const size_t min_part = (size_t)1 << 20;
    const int n = (int)std::max<size_t>(1, std::min<size_t>(workers.size() + 1, n_bytes / min_part));
    if (n == 1) {
      std::memcpy(d, sp, n_bytes);
      return;
    }
    const size_t p = (n_bytes / n + 4095) & ~(size_t)4095;
    {
      std::lock_guard<std::mutex> lk(mu);
      dst = static_cast<char*>(d);
      src = static_cast<const char*>(sp);
      bytes = n_bytes;
      part = p;
      nparts = n;
      pending = (int)workers.size();
      ++gen;
    }
    go.notify_all();
    std::memcpy(d, sp, std::min(n_bytes, p));
    std::unique_lock<std::mutex> lk(mu);
    done.wait(lk, [&] { return pending == 0; });
  }
  ~CopyPool() {
    {
      std::lock_guard<std::mutex> lk(mu);
      stop = true;
    }
    go.notify_all();
    for (std::thread& th : workers) th.join();
  }
};

struct Loader {
  int device = 0;
  size_t slot_bytes = 0;
  void* host[2] = {nullptr, nullptr};  // pinned
  void* dev[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  int slot = 0;
  uint64_t source_bytes = 0;  // PTQ1_0 bytes uploaded so far
  CopyPool pool;              // host copy of a slice
};

static void loader_free(Loader* L) {
  for (int i = 0; i < 2; ++i) {
    if (L->ev[i]) (void)hipEventDestroy(L->ev[i]);
    if (L->dev[i]) (void)hipFree(L->dev[i]);
    if (L->host[i]) (void)hipHostFree(L->host[i]);
  }
  delete L;
}

}  // namespace btfhip

using btfhip::Loader;
using btfhip::fail;

extern "C" {

int btf_hip_loader_create(uint64_t staging_bytes, btf_loader_t* out) {
  if (!out) return fail(BTF_ERR_ARGS, "loader: null argument");
  *out = nullptr;
  if (staging_bytes < 28 || staging_bytes > (1ull << 32))
    return fail(BTF_ERR_ARGS, "loader: staging slot must hold at least one block and be at most 4 GiB");
  const btfhip::DevState* ds = btfhip::current_state();
  if (!ds) return BTF_ERR_NOT_INIT;
  Loader* L = new Loader();
  (void)hipGetDevice(&L->device);
  L->slot_bytes = (size_t)staging_bytes;
  for (int i = 0; i < 2; ++i) {
    if (hipHostMalloc(&L->host[i], L->slot_bytes, hipHostMallocDefault) != hipSuccess ||
        hipMalloc(&L->dev[i], L->slot_bytes) != hipSuccess ||
        hipEventCreateWithFlags(&L->ev[i], hipEventDisableTiming) != hipSuccess) {
      btfhip::loader_free(L);
      return fail(BTF_ERR_LAUNCH, "loader: staging allocation failed");
    }
  }
  L->pool.start((int)std::max(1u, std::min(16u, std::thread::hardware_concurrency())) - 1);
  *out = L;
  return BTF_OK;
}

int btf_hip_loader_upload_ptq1_0(btf_loader_t h, const uint8_t* src, int64_t N, int64_t K, uint8_t* codes,
                                 uint16_t* scales, btf_stream_t stream) {
  Loader* L = static_cast<Loader*>(h);
  if (!L) return fail(BTF_ERR_ARGS, "loader: null loader");
  if (N <= 0) return BTF_OK;
  if (!src || !codes || !scales) return fail(BTF_ERR_ARGS, "loader: null pointer");
  if (K <= 0 || K % 128) return fail(BTF_ERR_ARGS, "loader: K must be a positive multiple of 128");
  if ((reinterpret_cast<uintptr_t>(codes) & 15) || (reinterpret_cast<uintptr_t>(scales) & 1))
    return fail(BTF_ERR_ARGS, "loader: codes must be 16-byte and scales 2-byte aligned");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != L->device)
    return fail(BTF_ERR_ARGS, "loader: upload on a device other than the loader's");
  const btfhip::DevState* ds = btfhip::current_state();
  if (!ds) return BTF_ERR_NOT_INIT;
  const int64_t nb = K / 128;               // blocks per row
  const size_t row_bytes = (size_t)nb * 28;  // PTQ1_0 bytes per row
  if (row_bytes > L->slot_bytes) return fail(BTF_ERR_ARGS, "loader: a row is larger than a staging slot");
  const int64_t rows_per = (int64_t)(L->slot_bytes / row_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int64_t r0 = 0; r0 < N; r0 += rows_per) {
    const int64_t rows = std::min(rows_per, N - r0);
    const size_t bytes = (size_t)rows * row_bytes;
    const int s = L->slot;
    L->slot ^= 1;
    // the slot's previous slice has been copied and repacked
    if (hipEventSynchronize(L->ev[s]) != hipSuccess) return fail(BTF_ERR_LAUNCH, "loader: staging wait failed");
    L->pool.copy(L->host[s], src + (size_t)r0 * row_bytes, bytes);
    if (hipMemcpyAsync(L->dev[s], L->host[s], bytes, hipMemcpyHostToDevice, st) != hipSuccess)
      return fail(BTF_ERR_LAUNCH, "loader: staging copy failed");
    const int rc = btfhip::repack(static_cast<const uint8_t*>(L->dev[s]), rows * nb, codes + r0 * (K / 4),
                                  scales + r0 * nb, st, *ds);
    if (rc != BTF_OK) return rc;
    if (hipEventRecord(L->ev[s], st) != hipSuccess) return fail(BTF_ERR_LAUNCH, "loader: event record failed");
    L->source_bytes += bytes;
  }
  return BTF_OK;
}

int btf_hip_loader_finish(btf_loader_t h, uint64_t* source_bytes) {
  Loader* L = static_cast<Loader*>(h);
  if (!L) return fail(BTF_ERR_ARGS, "loader: null loader");
  for (int i = 0; i < 2; ++i)
    if (hipEventSynchronize(L->ev[i]) != hipSuccess) return fail(BTF_ERR_LAUNCH, "loader: wait failed");
  if (source_bytes) *source_bytes = L->source_bytes;
  return BTF_OK;
}

int btf_hip_loader_destroy(btf_loader_t h) {
  Loader* L = static_cast<Loader*>(h);
  if (!L) return BTF_OK;
  for (int i = 0; i < 2; ++i)
    if (L->ev[i]) (void)hipEventSynchronize(L->ev[i]);
  btfhip::loader_free(L);
  return BTF_OK;
}

int btf_hip_gguf_plan(btf_gguf_t h, uint64_t staging_bytes, btf_pack_plan* out) {
  if (!h || !out) return fail(BTF_ERR_ARGS, "plan: null argument");
  btf_gguf_header hd;
  if (const int rc = btf_hip_gguf_info(h, &hd)) return rc;
  btf_pack_plan p;
  std::memset(&p, 0, sizeof p);
  for (int64_t i = 0; i < hd.n_tensors; ++i) {
    btf_gguf_tensor t;
    if (const int rc = btf_hip_gguf_tensor(h, i, &t)) return rc;
    if (t.type == 143 && t.n_dims == 2) {  // PTQ1_0 matrix: ne[0] = K (contiguous), ne[1] = N rows
      const uint64_t K = (uint64_t)t.ne[0], N = (uint64_t)t.ne[1];
      const uint64_t cb = N * (K / 4), sb = N * (K / 128) * 2;
      ++p.n_matrices;
      p.codes_bytes += cb;
      p.scales_bytes += sb;
      p.arena_bytes += (cb + 255) / 256 * 256 + (sb + 255) / 256 * 256;
      p.source_bytes += t.bytes;
    } else {
      p.other_bytes += t.bytes;
    }
  }
  p.staging_host_bytes = 2 * staging_bytes;
  p.staging_device_bytes = 2 * staging_bytes;
  *out = p;
  return BTF_OK;
}

}  // extern "C"
