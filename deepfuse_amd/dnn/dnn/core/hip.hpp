// dnn/core/hip.hpp -- device context and stream contract of the drop-in.
//
// Mirrors the reference's Cuda class and StreamGuard (dnn/core/cuda.cuh:23-71,
// dnn/core/cuda.cu:26-172): constructing Hip(device) selects the device and
// forces context creation, registers itself as the calling thread's current
// instance, and the thread-local stream defaults to the legacy default
// stream.  Unlike the reference, every kernel the drop-in launches goes to
// Hip::stream().  `Cuda` is kept as an alias so reference callers compile.
#pragma once

#include <hip/hip_runtime.h>

#include <iostream>
#include <string>
#include <vector>

namespace dnn {

// One GPU's properties (the reference's Device, dnn/core/device.cuh:12-37).
// num_sm() reports compute units, the CDNA counterpart of SMs.
class Device {
public:
    explicit Device(int device_id = 0);
    int id() const { return id_; }
    // marketing name; the architecture when the driver reports none
    std::string name() const { return props_.name[0] ? props_.name : std::string("AMD ") + props_.gcnArchName; }
    std::string architecture_name() const { return props_.gcnArchName; }
    int compute_capability_major() const { return props_.major; }
    int compute_capability_minor() const { return props_.minor; }
    size_t total_memory_bytes() const { return props_.totalGlobalMem; }
    size_t available_memory_bytes() const;
    int num_sm() const { return props_.multiProcessorCount; }
    float clock_ghz() const { return props_.clockRate * 1e-6f; }
    void dump_info(std::ostream& os = std::cout) const;

private:
    int id_;
    hipDeviceProp_t props_;
};

class Hip {
public:
    explicit Hip(int device_id = 0);
    ~Hip();
    Hip(const Hip&) = delete;
    Hip& operator=(const Hip&) = delete;

    int id() const { return id_; }
    static Hip& current();  // throws when the calling thread has none
    static const std::vector<Device>& get_devices();
    void dump_info(std::ostream& os = std::cout) const;

    // stream multiplexing (thread-local; nullptr selects the legacy default
    // stream, as in the reference)
    static void set_stream(hipStream_t stream);
    static hipStream_t stream();

private:
    int id_;
};

class StreamGuard {
public:
    explicit StreamGuard(hipStream_t new_stream);
    ~StreamGuard();
    StreamGuard(const StreamGuard&) = delete;
    StreamGuard& operator=(const StreamGuard&) = delete;

private:
    hipStream_t previous_;
};

using Cuda = Hip;  // reference spelling (dnn/core/cuda.cuh:23)

}  // namespace dnn
