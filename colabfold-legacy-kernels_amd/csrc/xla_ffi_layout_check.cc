// Compile-time check that xla_ffi_abi.h matches XLA's own C ABI header byte for byte. Built
// (syntax-only, no code) by build.py when FFI_INCLUDE names a directory holding
// xla/ffi/api/c_api.h -- the same gate as the reference's scripts/build_kernels.sh:44-51.
#include <cstddef>

#include "xla/ffi/api/c_api.h"
#include "xla_ffi_abi.h"

namespace x = clk::xffi;

#define CLK_SAME_SIZE(A, B) static_assert(sizeof(A) == sizeof(B), "size of " #A)
#define CLK_SAME_OFFSET(A, fa, B, fb) \
    static_assert(offsetof(A, fa) == offsetof(B, fb), "offset of " #A "::" #fa)

static_assert(XLA_FFI_API_MAJOR == x::kApiMajor && XLA_FFI_API_MINOR == x::kApiMinor,
              "XLA FFI API version");

CLK_SAME_SIZE(XLA_FFI_Extension_Base, x::ExtensionBase);
CLK_SAME_OFFSET(XLA_FFI_Extension_Base, type, x::ExtensionBase, type);
CLK_SAME_OFFSET(XLA_FFI_Extension_Base, next, x::ExtensionBase, next);

CLK_SAME_SIZE(XLA_FFI_Error_Create_Args, x::ErrorCreateArgs);
CLK_SAME_OFFSET(XLA_FFI_Error_Create_Args, message, x::ErrorCreateArgs, message);
CLK_SAME_OFFSET(XLA_FFI_Error_Create_Args, errc, x::ErrorCreateArgs, errc);

CLK_SAME_SIZE(XLA_FFI_Stream_Get_Args, x::StreamGetArgs);
CLK_SAME_OFFSET(XLA_FFI_Stream_Get_Args, ctx, x::StreamGetArgs, ctx);
CLK_SAME_OFFSET(XLA_FFI_Stream_Get_Args, stream, x::StreamGetArgs, stream);

CLK_SAME_SIZE(XLA_FFI_Api_Version, x::ApiVersion);
CLK_SAME_OFFSET(XLA_FFI_Api, api_version, x::Api, api_version);
CLK_SAME_OFFSET(XLA_FFI_Api, XLA_FFI_Error_Create, x::Api, error_create);
CLK_SAME_OFFSET(XLA_FFI_Api, XLA_FFI_Stream_Get, x::Api, stream_get);

CLK_SAME_SIZE(XLA_FFI_Buffer, x::Buffer);
CLK_SAME_OFFSET(XLA_FFI_Buffer, dtype, x::Buffer, dtype);
CLK_SAME_OFFSET(XLA_FFI_Buffer, data, x::Buffer, data);
CLK_SAME_OFFSET(XLA_FFI_Buffer, rank, x::Buffer, rank);
CLK_SAME_OFFSET(XLA_FFI_Buffer, dims, x::Buffer, dims);

CLK_SAME_SIZE(XLA_FFI_Args, x::Args);
CLK_SAME_OFFSET(XLA_FFI_Args, size, x::Args, size);
CLK_SAME_OFFSET(XLA_FFI_Args, types, x::Args, types);
CLK_SAME_OFFSET(XLA_FFI_Args, args, x::Args, args);
CLK_SAME_SIZE(XLA_FFI_Rets, x::Rets);
CLK_SAME_OFFSET(XLA_FFI_Rets, rets, x::Rets, rets);

CLK_SAME_SIZE(XLA_FFI_ByteSpan, x::ByteSpan);
CLK_SAME_SIZE(XLA_FFI_Scalar, x::Scalar);
CLK_SAME_OFFSET(XLA_FFI_Scalar, value, x::Scalar, value);
CLK_SAME_SIZE(XLA_FFI_Attrs, x::Attrs);
CLK_SAME_OFFSET(XLA_FFI_Attrs, types, x::Attrs, types);
CLK_SAME_OFFSET(XLA_FFI_Attrs, names, x::Attrs, names);
CLK_SAME_OFFSET(XLA_FFI_Attrs, attrs, x::Attrs, attrs);

CLK_SAME_OFFSET(XLA_FFI_CallFrame, api, x::CallFrame, api);
CLK_SAME_OFFSET(XLA_FFI_CallFrame, ctx, x::CallFrame, ctx);
CLK_SAME_OFFSET(XLA_FFI_CallFrame, stage, x::CallFrame, stage);
CLK_SAME_OFFSET(XLA_FFI_CallFrame, args, x::CallFrame, args);
CLK_SAME_OFFSET(XLA_FFI_CallFrame, rets, x::CallFrame, rets);
CLK_SAME_OFFSET(XLA_FFI_CallFrame, attrs, x::CallFrame, attrs);

CLK_SAME_OFFSET(XLA_FFI_Metadata, api_version, x::Metadata, api_version);
CLK_SAME_OFFSET(XLA_FFI_Metadata, traits, x::Metadata, traits);
CLK_SAME_OFFSET(XLA_FFI_Metadata_Extension, metadata, x::MetadataExtension, metadata);

static_assert(XLA_FFI_DataType_F16 == x::kF16 && XLA_FFI_DataType_BF16 == x::kBF16 &&
                  XLA_FFI_DataType_F32 == x::kF32 && XLA_FFI_DataType_U8 == x::kU8 &&
                  XLA_FFI_DataType_S64 == x::kS64,
              "dtype codes");
static_assert(XLA_FFI_Error_Code_INVALID_ARGUMENT == x::kInvalidArgument &&
                  XLA_FFI_Error_Code_INTERNAL == x::kInternal,
              "error codes");
static_assert(XLA_FFI_ExecutionStage_EXECUTE == x::kExecute, "execution stage");
static_assert(XLA_FFI_Extension_Metadata == x::kExtensionMetadata, "metadata extension");
static_assert(XLA_FFI_ArgType_BUFFER == x::kArgBuffer && XLA_FFI_AttrType_SCALAR == x::kAttrScalar,
              "arg and attribute kinds");
