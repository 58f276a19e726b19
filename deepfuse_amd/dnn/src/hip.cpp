// Hip context and stream guard (dnn/core/cuda.cu:26-172 in the reference).
#include "dnn/core/hip.hpp"

#include <stdexcept>

#include "dnn/utils/common.hpp"

namespace dnn {

namespace {
thread_local Hip* g_current = nullptr;
thread_local hipStream_t g_stream = nullptr;
}  // namespace

Device::Device(int device_id) : id_(device_id) { CHECK_HIP_EX(hipGetDeviceProperties(&props_, id_)); }

size_t Device::available_memory_bytes() const {
    int prev = 0;
    CHECK_HIP_EX(hipGetDevice(&prev));
    CHECK_HIP_EX(hipSetDevice(id_));
    size_t free_b = 0, total_b = 0;
    const hipError_t e = hipMemGetInfo(&free_b, &total_b);
    CHECK_HIP_EX(hipSetDevice(prev));
    CHECK_HIP_EX(e);
    return free_b;
}

void Device::dump_info(std::ostream& os) const {
    os << "HIP Device " << id_ << ": " << name() << " (" << architecture_name() << "), " << num_sm() << " CUs, "
       << (total_memory_bytes() >> 20) << " MiB, " << clock_ghz() << " GHz";
}

Hip::Hip(int device_id) : id_(device_id) {
    CHECK_HIP_EX(hipSetDevice(id_));
    CHECK_HIP_EX(hipFree(nullptr));  // force context creation
    g_current = this;
}

Hip::~Hip() {
    if (g_current == this) g_current = nullptr;
}

Hip& Hip::current() {
    if (!g_current) throw std::runtime_error("No current Hip instance set.");
    return *g_current;
}

const std::vector<Device>& Hip::get_devices() {
    static const std::vector<Device> cache = [] {
        int count = 0;
        CHECK_HIP_EX(hipGetDeviceCount(&count));
        std::vector<Device> out;
        for (int i = 0; i < count; ++i) out.emplace_back(i);
        return out;
    }();
    return cache;
}

void Hip::dump_info(std::ostream& os) const {
    os << "[HIP System Summary]\n";
    for (const auto& d : get_devices()) {
        d.dump_info(os);
        os << "\n";
    }
}

void Hip::set_stream(hipStream_t stream) { g_stream = stream; }

hipStream_t Hip::stream() { return g_stream ? g_stream : hipStreamLegacy; }

StreamGuard::StreamGuard(hipStream_t new_stream) : previous_(Hip::stream()) { Hip::set_stream(new_stream); }

StreamGuard::~StreamGuard() { Hip::set_stream(previous_); }

}  // namespace dnn
