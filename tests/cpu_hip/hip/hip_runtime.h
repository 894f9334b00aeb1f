// A CPU stand-in for the HIP runtime API that pk_gpu_runtime.hip uses, for
// the registry stress test (test_registry_cpu.py): device memory is host
// memory, and every asynchronous operation is queued on its stream and runs
// only when the stream (or the device) is synchronised, as on a GPU, so a
// copy freed while queued work still reads it is a use after free that
// ThreadSanitizer reports.  Declarations only; cpu_hip.cpp implements them.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>

#define __device__
#define __host__
#define __global__
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) (&(x))

typedef enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorNotSupported = 801,
    hipErrorUnknown = 999,
} hipError_t;

typedef enum hipMemcpyKind {
    hipMemcpyHostToHost = 0,
    hipMemcpyHostToDevice = 1,
    hipMemcpyDeviceToHost = 2,
    hipMemcpyDeviceToDevice = 3,
    hipMemcpyDefault = 4,
} hipMemcpyKind;

typedef enum hipStreamCaptureStatus {
    hipStreamCaptureStatusNone = 0,
    hipStreamCaptureStatusActive = 1,
    hipStreamCaptureStatusInvalidated = 2,
} hipStreamCaptureStatus;

#define hipStreamDefault 0
#define hipStreamNonBlocking 1

struct ihipStream_t;
typedef ihipStream_t* hipStream_t;

struct hipDeviceProp_t {
    char name[256];
    char gcnArchName[256];
    int multiProcessorCount;
};

hipError_t hipGetDeviceCount(int* n);
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int device);
hipError_t hipSetDevice(int device);
hipError_t hipGetDevice(int* device);
hipError_t hipGetSymbolAddress(void** out, const void* symbol);
hipError_t hipMalloc(void** p, size_t bytes);
hipError_t hipFree(void* p);
hipError_t hipMemcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind);
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t s);
hipError_t hipMemcpy2DAsync(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                            size_t rows, hipMemcpyKind kind, hipStream_t s);
hipError_t hipMemsetAsync(void* dst, int value, size_t bytes, hipStream_t s);
hipError_t hipStreamCreate(hipStream_t* s);
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus* status);
hipError_t hipDeviceSynchronize();
hipError_t hipGetLastError();
const char* hipGetErrorString(hipError_t e);

// Test hooks.  Queue work on a stream (NULL: the null stream), run at its
// next synchronisation (the kernel stand-ins use it).  Give the calling
// thread a role, and count the explicit hipDeviceSynchronize calls made from
// threads of a role (device-wide work that a caller's thread should never do).
void cpu_hip_enqueue(hipStream_t s, std::function<void()> work);
void cpu_hip_set_role(int role);
long cpu_hip_device_syncs(int role);
