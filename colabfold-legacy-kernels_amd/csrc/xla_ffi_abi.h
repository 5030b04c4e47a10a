// The subset of the XLA FFI C ABI (xla/ffi/api/c_api.h, API version 0.1 as shipped with
// jax 0.6) that the custom-call handlers in xla_ffi.cpp use, declared here because the XLA
// headers are not part of this build's toolchain. The struct layouts must match XLA's byte for
// byte: xla_ffi_layout_check.cc static-asserts every offset and size below against the real
// header whenever FFI_INCLUDE points at one (the same gate as the reference's
// scripts/build_kernels.sh:44-58).
//
// Only these members of XLA_FFI_Api are read: XLA_FFI_Error_Create (to return an error) and
// XLA_FFI_Stream_Get (the platform stream, a hipStream_t on ROCm). Contexts such as the device
// ordinal are fetched through the API by the handler, not passed in the call frame, so the
// handlers need nothing else.
#pragma once

#include <cstddef>
#include <cstdint>

namespace clk {
namespace xffi {

enum ExtensionType : int32_t { kExtensionMetadata = 1 };

struct ExtensionBase {
    size_t struct_size;
    ExtensionType type;
    ExtensionBase* next;
};

enum ExecutionStage : int32_t { kInstantiate = 0, kPrepare = 1, kInitialize = 2, kExecute = 3 };

enum DataType : int32_t {
    kInvalid = 0, kPred = 1, kS8 = 2, kS16 = 3, kS32 = 4, kS64 = 5, kU8 = 6, kU16 = 7, kU32 = 8,
    kU64 = 9, kF16 = 10, kF32 = 11, kF64 = 12, kC64 = 15, kBF16 = 16, kToken = 17, kC128 = 18
};

enum ErrorCode : int32_t { kOk = 0, kInvalidArgument = 3, kUnimplemented = 12, kInternal = 13 };

enum ArgType : int32_t { kArgBuffer = 1 };
enum RetType : int32_t { kRetBuffer = 1 };
enum AttrType : int32_t { kAttrArray = 1, kAttrDictionary = 2, kAttrScalar = 3, kAttrString = 4 };

struct Error;  // opaque
struct ExecutionContext;  // opaque
struct Future;  // opaque

struct ErrorCreateArgs {
    size_t struct_size;
    ExtensionBase* extension_start;
    const char* message;
    ErrorCode errc;
};
typedef Error* ErrorCreateFn(ErrorCreateArgs* args);

struct StreamGetArgs {
    size_t struct_size;
    ExtensionBase* extension_start;
    ExecutionContext* ctx;
    void* stream;  // out
};
typedef Error* StreamGetFn(StreamGetArgs* args);

struct ApiVersion {
    size_t struct_size;
    ExtensionBase* extension_start;
    int major_version;
    int minor_version;
};

// Leading members of XLA_FFI_Api, up to the last one used here.
struct Api {
    size_t struct_size;
    ExtensionBase* extension_start;
    ApiVersion api_version;
    void* internal_api;
    ErrorCreateFn* error_create;
    void* error_get_message;
    void* error_destroy;
    void* handler_register;
    StreamGetFn* stream_get;
};

struct Buffer {
    size_t struct_size;
    ExtensionBase* extension_start;
    DataType dtype;
    void* data;
    int64_t rank;
    int64_t* dims;
};

struct Args {
    size_t struct_size;
    ExtensionBase* extension_start;
    int64_t size;
    ArgType* types;
    void** args;
};

struct Rets {
    size_t struct_size;
    ExtensionBase* extension_start;
    int64_t size;
    RetType* types;
    void** rets;
};

struct ByteSpan {
    const char* ptr;
    size_t len;
};

struct Scalar {
    DataType dtype;
    void* value;
};

struct Attrs {
    size_t struct_size;
    ExtensionBase* extension_start;
    int64_t size;
    AttrType* types;
    ByteSpan** names;
    void** attrs;
};

struct CallFrame {
    size_t struct_size;
    ExtensionBase* extension_start;
    const Api* api;
    ExecutionContext* ctx;
    ExecutionStage stage;
    Args args;
    Rets rets;
    Attrs attrs;
    Future* future;
};

typedef uint32_t HandlerTraits;
constexpr HandlerTraits kCommandBufferCompatible = 1u << 0;

struct Metadata {
    size_t struct_size;
    ApiVersion api_version;
    HandlerTraits traits;
};

struct MetadataExtension {
    ExtensionBase extension_base;
    Metadata* metadata;
};

constexpr int kApiMajor = 0;
constexpr int kApiMinor = 1;

}  // namespace xffi
}  // namespace clk
