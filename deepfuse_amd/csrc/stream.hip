// stream.hip -- layer weight streaming: a ring of device slots filled from
// pinned host memory by hipMemcpyAsync on the streamer's own two copy
// streams (consecutive loads alternate), ordered against the compute stream
// with events in both directions:
//   load(l)    : the calling thread waits until the event recorded when the
//                slot's previous contents were released has completed, then
//                enqueues the copy and records loaded[s] on its copy stream;
//   wait(s)    : the compute stream waits for loaded[s];
//   release(s) : records released[s] on the compute stream after the last
//                launch that reads the slot.
// With S slots and loads issued S-2 layers ahead (load l+S-2 right after
// layer l's launches), the thread blocks until layer l-2 has finished while
// layers l-1 and l are queued, and the copies run S-2 layers ahead of the
// kernels that read them.
//
// Two copy streams: a load is enqueued when its slot frees, which at the
// compute pace often finds the copy engine idle, and a copy started on an
// idle engine took about 90 us longer than one queued behind another
// (30.72 MB copies: 0.54 ms back to back, gaps of 93-121 us between
// host-paced ones).  That made the streamed config-5 step copy-bound (about
// 0.63 ms of copy per layer against 0.56 ms of compute).  With consecutive
// loads on alternating streams one copy's start overlaps the other's
// transfer.
//
// The reference describes this as layer-serialized execution
// (README.md:212-226) but implements only the host side of it: pinned
// cudaHostAlloc buffers, per-slot streams and cudaMemcpyAsync in its NVMe
// loader (apps/host-multi/NVMeLoader_Linux.hpp:20-26,64-71,123-125).  Here
// the same pieces feed the fp8 GEMMs: each slot holds one layer's e4m3
// weight codes.
#include <hip/hip_runtime.h>

#include <new>
#include <vector>

#include "df_common.hpp"

namespace dfk {

constexpr int kMaxSlots = 64;

constexpr size_t kSlotAlign = 4096;

enum SlotState : int { kEmpty = 0, kLoaded = 1, kReleased = 2 };

}  // namespace dfk

struct df_streamer_s {
    int device = -1;
    int slots = 0;
    size_t slot_bytes = 0;
    uint8_t* dev = nullptr;
    hipStream_t copy[2] = {};
    unsigned loads = 0;  // loads issued: load i goes to copy[i % 2]
    hipEvent_t loaded[dfk::kMaxSlots] = {};
    hipEvent_t released[dfk::kMaxSlots] = {};
    int state[dfk::kMaxSlots] = {};
    int next = 0;
    // timing mode: events recorded on the copy stream right before and after
    // each copy; a slot's pair is read into the log once that copy is known
    // to be complete (its slot is loaded again, or the log is read)
    bool timing = false;
    hipEvent_t t_start[dfk::kMaxSlots] = {};
    hipEvent_t t_end[dfk::kMaxSlots] = {};
    bool t_pending[dfk::kMaxSlots] = {};
    size_t t_bytes[dfk::kMaxSlots] = {};
    hipEvent_t t_origin = nullptr;  // recorded just before the first timed copy since the log was read
    bool have_origin = false;
    std::vector<float> log_start, log_end;
    std::vector<size_t> log_bytes;
};

using namespace dfk;

#define DF_HIP(call, what)                                                                      \
    do {                                                                                        \
        const hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) {                                                                 \
            set_error("%s: HIP error %d (%s)", what, (int)e_, hipGetErrorString(e_));           \
            return DF_ERR_HIP;                                                                  \
        }                                                                                       \
    } while (0)

extern "C" int df_host_alloc(size_t bytes, void** host_ptr) {
    clear_error();
    DF_CHECK(host_ptr, DF_ERR_INVALID, "df_host_alloc: host_ptr is NULL");
    *host_ptr = nullptr;
    if (bytes == 0) return DF_OK;
    DF_HIP(hipHostMalloc(host_ptr, bytes, hipHostMallocDefault), "df_host_alloc");
    return DF_OK;
}

extern "C" int df_host_free(void* host_ptr) {
    clear_error();
    if (host_ptr) DF_HIP(hipHostFree(host_ptr), "df_host_free");
    return DF_OK;
}

static void destroy_streamer(df_streamer_s* s) {
    if (!s) return;
    for (hipStream_t c : s->copy)
        if (c) (void)hipStreamSynchronize(c);
    for (int i = 0; i < kMaxSlots; ++i) {
        if (s->loaded[i]) (void)hipEventDestroy(s->loaded[i]);
        if (s->released[i]) (void)hipEventDestroy(s->released[i]);
        if (s->t_start[i]) (void)hipEventDestroy(s->t_start[i]);
        if (s->t_end[i]) (void)hipEventDestroy(s->t_end[i]);
    }
    if (s->t_origin) (void)hipEventDestroy(s->t_origin);  // its own event (created with the timing pairs)
    for (hipStream_t c : s->copy)
        if (c) (void)hipStreamDestroy(c);
    if (s->dev) (void)hipFree(s->dev);
    delete s;
}

extern "C" int df_streamer_create(int slots, size_t slot_bytes, df_streamer_s** out) {
    clear_error();
    DF_CHECK(out, DF_ERR_INVALID, "df_streamer_create: out is NULL");
    *out = nullptr;
    DF_CHECK(slots >= 2 && slots <= kMaxSlots, DF_ERR_INVALID, "df_streamer_create: slots=%d not in [2, %d]",
             slots, kMaxSlots);
    DF_CHECK(slot_bytes > 0, DF_ERR_INVALID, "df_streamer_create: slot_bytes is 0");
    df_streamer_s* s = new (std::nothrow) df_streamer_s();
    DF_CHECK(s, DF_ERR_INVALID, "df_streamer_create: out of host memory");
    s->slots = slots;
    s->slot_bytes = (slot_bytes + kSlotAlign - 1) / kSlotAlign * kSlotAlign;
    hipError_t e = hipGetDevice(&s->device);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&s->dev), s->slot_bytes * (size_t)slots);
    // default priority, non-blocking with respect to the null stream
    for (hipStream_t& c : s->copy)
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&c, hipStreamNonBlocking);
    for (int i = 0; i < slots && e == hipSuccess; ++i) {
        e = hipEventCreateWithFlags(&s->loaded[i], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&s->released[i], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        set_error("df_streamer_create: HIP error %d (%s)", (int)e, hipGetErrorString(e));
        destroy_streamer(s);
        return DF_ERR_HIP;
    }
    *out = s;
    return DF_OK;
}

extern "C" int df_streamer_destroy(df_streamer_s* s) {
    clear_error();
    destroy_streamer(s);
    return DF_OK;
}

extern "C" int df_streamer_copy_stream(df_streamer_s* s, int which, void** stream) {
    clear_error();
    DF_CHECK(s && stream, DF_ERR_INVALID, "df_streamer_copy_stream: NULL argument");
    DF_CHECK(which == 0 || which == 1, DF_ERR_INVALID, "df_streamer_copy_stream: which=%d is not 0 or 1", which);
    *stream = s->copy[which];
    return DF_OK;
}

extern "C" int df_streamer_slot(df_streamer_s* s, int slot, void** dev_ptr) {
    clear_error();
    DF_CHECK(s && dev_ptr, DF_ERR_INVALID, "df_streamer_slot: NULL argument");
    DF_CHECK(slot >= 0 && slot < s->slots, DF_ERR_INVALID, "df_streamer_slot: slot %d out of range", slot);
    *dev_ptr = s->dev + (size_t)slot * s->slot_bytes;
    return DF_OK;
}

// Moves slot k's timed copy into the log (start and end in ms after the
// origin event, which was recorded just before the first timed copy since
// the log was last read); waits for that copy to complete.
static int log_slot(df_streamer_s* s, int k, const char* what) {
    if (!s->t_pending[k]) return DF_OK;
    DF_HIP(hipEventSynchronize(s->t_end[k]), what);
    DF_HIP(hipEventSynchronize(s->t_origin), what);  // it may sit on the other copy stream
    float a = 0.0f, b = 0.0f;
    DF_HIP(hipEventElapsedTime(&a, s->t_origin, s->t_start[k]), what);
    DF_HIP(hipEventElapsedTime(&b, s->t_origin, s->t_end[k]), what);
    s->log_start.push_back(a);
    s->log_end.push_back(b);
    s->log_bytes.push_back(s->t_bytes[k]);
    s->t_pending[k] = false;
    return DF_OK;
}

extern "C" int df_streamer_set_timing(df_streamer_s* s, int on) {
    clear_error();
    DF_CHECK(s, DF_ERR_INVALID, "df_streamer_set_timing: streamer is NULL");
    if (on && !s->t_origin) {
        DF_HIP(hipEventCreate(&s->t_origin), "df_streamer_set_timing");
        for (int i = 0; i < s->slots; ++i) {
            DF_HIP(hipEventCreate(&s->t_start[i]), "df_streamer_set_timing");
            DF_HIP(hipEventCreate(&s->t_end[i]), "df_streamer_set_timing");
        }
    }
    s->timing = on != 0;
    return DF_OK;
}

extern "C" int df_streamer_copy_log(df_streamer_s* s, float* start_ms, float* end_ms, int capacity, int* count) {
    clear_error();
    DF_CHECK(s && count && (capacity == 0 || (start_ms && end_ms)), DF_ERR_INVALID,
             "df_streamer_copy_log: NULL argument");
    DF_CHECK(capacity >= 0, DF_ERR_INVALID, "df_streamer_copy_log: capacity < 0");
    // every timed copy still in flight completes first, in load order
    for (int j = 0; j < s->slots; ++j) {
        const int k = (s->next + j) % s->slots;
        if (int rc = log_slot(s, k, "df_streamer_copy_log")) return rc;
    }
    const int n = (int)s->log_start.size();
    for (int i = 0; i < n && i < capacity; ++i) {
        start_ms[i] = s->log_start[i];
        end_ms[i] = s->log_end[i];
    }
    *count = n;
    if (capacity >= n) {  // every entry handed out: start a new log
        s->log_start.clear();
        s->log_end.clear();
        s->log_bytes.clear();
        s->have_origin = false;
    }
    return DF_OK;
}

extern "C" int df_streamer_load(df_streamer_s* s, const void* host_src, size_t bytes, int* slot, void** dev_ptr) {
    clear_error();
    DF_CHECK(s && host_src && slot, DF_ERR_INVALID, "df_streamer_load: NULL argument");
    DF_CHECK(bytes <= s->slot_bytes, DF_ERR_INVALID, "df_streamer_load: %zu bytes exceed the slot size %zu", bytes,
             s->slot_bytes);
    const int k = s->next;
    DF_CHECK(s->state[k] != kLoaded, DF_ERR_INVALID,
             "df_streamer_load: slot %d is still in use (df_streamer_release was not called for it)", k);
    // The calling thread, not the copy engine, waits for the release: a copy
    // made to wait on the GPU for an event of the compute stream delays the
    // compute stream's own work (measured: 81.5 ms instead of 65.5 ms for a
    // 96-layer sweep whose kernels alone take 57.6 ms).
    if (s->state[k] == kReleased) {
        DF_HIP(hipEventSynchronize(s->released[k]), "df_streamer_load");
        // the slot's previous copy ran on the other copy stream, so stream
        // order does not keep it ahead of this one; a caller that waited on
        // it before releasing the slot has made it complete already (then
        // this returns at once), one that did not is covered here
        DF_HIP(hipEventSynchronize(s->loaded[k]), "df_streamer_load");
    }
    if (int rc = log_slot(s, k, "df_streamer_load")) return rc;
    uint8_t* dst = s->dev + (size_t)k * s->slot_bytes;
    hipStream_t cs = s->copy[s->loads++ & 1u];
    if (s->timing) {
        if (!s->have_origin) DF_HIP(hipEventRecord(s->t_origin, cs), "df_streamer_load");
        s->have_origin = true;
        DF_HIP(hipEventRecord(s->t_start[k], cs), "df_streamer_load");
    }
    if (bytes) DF_HIP(hipMemcpyAsync(dst, host_src, bytes, hipMemcpyHostToDevice, cs), "df_streamer_load");
    DF_HIP(hipEventRecord(s->loaded[k], cs), "df_streamer_load");
    if (s->timing) {
        DF_HIP(hipEventRecord(s->t_end[k], cs), "df_streamer_load");
        s->t_pending[k] = true;
        s->t_bytes[k] = bytes;
    }
    s->state[k] = kLoaded;
    s->next = (k + 1) % s->slots;
    *slot = k;
    if (dev_ptr) *dev_ptr = dst;
    return DF_OK;
}

extern "C" int df_streamer_wait(df_streamer_s* s, int slot, void* stream) {
    clear_error();
    DF_CHECK(s, DF_ERR_INVALID, "df_streamer_wait: streamer is NULL");
    DF_CHECK(slot >= 0 && slot < s->slots, DF_ERR_INVALID, "df_streamer_wait: slot %d out of range", slot);
    DF_CHECK(s->state[slot] == kLoaded, DF_ERR_INVALID, "df_streamer_wait: slot %d holds no load", slot);
    DF_HIP(hipStreamWaitEvent(as_stream(stream), s->loaded[slot], 0), "df_streamer_wait");
    return DF_OK;
}

extern "C" int df_streamer_release(df_streamer_s* s, int slot, void* stream) {
    clear_error();
    DF_CHECK(s, DF_ERR_INVALID, "df_streamer_release: streamer is NULL");
    DF_CHECK(slot >= 0 && slot < s->slots, DF_ERR_INVALID, "df_streamer_release: slot %d out of range", slot);
    DF_CHECK(s->state[slot] == kLoaded, DF_ERR_INVALID, "df_streamer_release: slot %d holds no load", slot);
    DF_HIP(hipEventRecord(s->released[slot], as_stream(stream)), "df_streamer_release");
    s->state[slot] = kReleased;
    return DF_OK;
}
