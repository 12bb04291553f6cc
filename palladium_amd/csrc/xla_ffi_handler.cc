// jax.ffi entry point "palladium_hip_dispatch": one generic XLA FFI handler
// for every palladium_amd kernel, registered on the "cpu" platform, as the
// reference's native/ffi/palladium_ffi.cpp:110-209 is for Metal. Source,
// entry point, Pallas grid, workgroup size, threads per program instance
// (`lanes`) and math mode arrive as FFI attributes (baked into the HLO at
// trace time); buffers as RemainingArgs/RemainingRets. Everything else is
// the C ABI's ph_dispatch (include/palladium_hip.h): compile cache,
// host->device staging, launch, device->host copy, wait.
//
// "palladium_hip_dispatch_rocm" is the same handler for jax on ROCm: the
// buffers are already in HBM and the launch is ordered on XLA's own stream
// (ph_dispatch_device: no staging, no wait).
//
// Built only where the XLA FFI headers exist (`jax.ffi.include_dir()`):
//   python -m palladium_amd.build --ffi

#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "palladium_hip.h"
#include "xla/ffi/api/ffi.h"

namespace {

xla::ffi::Error PalladiumHipDispatch(std::string_view hip_source,
                                     std::string_view function_name,
                                     int64_t grid_x, int64_t grid_y,
                                     int64_t grid_z, int64_t block_x,
                                     int64_t lanes, int64_t math_mode,
                                     xla::ffi::RemainingArgs args,
                                     xla::ffi::RemainingRets rets) {
  if (math_mode < PH_MATH_SAFE || math_mode > PH_MATH_REPRODUCIBLE)
    return xla::ffi::Error::InvalidArgument(
        "palladium_hip_dispatch: math_mode out of range");
  std::vector<const void *> in_ptrs;
  std::vector<size_t> in_bytes;
  std::vector<void *> out_ptrs;
  std::vector<size_t> out_bytes;
  for (size_t i = 0; i < args.size(); ++i) {
    auto buf = args.get<xla::ffi::AnyBuffer>(i);
    if (!buf.has_value()) return buf.error();
    in_ptrs.push_back(buf->untyped_data());
    in_bytes.push_back(buf->size_bytes());
  }
  for (size_t i = 0; i < rets.size(); ++i) {
    auto buf = rets.get<xla::ffi::AnyBuffer>(i);
    if (!buf.has_value()) return buf.error();
    out_ptrs.push_back((*buf)->untyped_data());
    out_bytes.push_back((*buf)->size_bytes());
  }
  std::string name(function_name);
  char *err = nullptr;
  int rc = ph_dispatch(hip_source.data(), hip_source.size(), name.c_str(), grid_x,
                       grid_y, grid_z, block_x, lanes, math_mode, in_ptrs.data(),
                       in_bytes.data(), in_ptrs.size(), out_ptrs.data(),
                       out_bytes.data(), out_ptrs.size(), &err);
  if (rc != PH_OK) {
    std::string msg = err ? err : "ph_dispatch failed";
    ph_free_error(err);
    if (rc == PH_ERR_INVALID_ARGUMENT)
      return xla::ffi::Error::InvalidArgument(msg);
    return xla::ffi::Error::Internal(msg);
  }
  return xla::ffi::Error::Success();
}

}  // namespace

XLA_FFI_DEFINE_HANDLER_SYMBOL(palladium_hip_dispatch, PalladiumHipDispatch,
                              xla::ffi::Ffi::Bind()
                                  .Attr<std::string_view>("hip_source")
                                  .Attr<std::string_view>("function_name")
                                  .Attr<int64_t>("grid_x")
                                  .Attr<int64_t>("grid_y")
                                  .Attr<int64_t>("grid_z")
                                  .Attr<int64_t>("block_x")
                                  .Attr<int64_t>("lanes")
                                  .Attr<int64_t>("math_mode")
                                  .RemainingArgs()
                                  .RemainingRets());

namespace {

xla::ffi::Error PalladiumHipDispatchRocm(hipStream_t stream,
                                         std::string_view hip_source,
                                         std::string_view function_name,
                                         int64_t grid_x, int64_t grid_y,
                                         int64_t grid_z, int64_t block_x,
                                         int64_t lanes, int64_t math_mode,
                                         xla::ffi::RemainingArgs args,
                                         xla::ffi::RemainingRets rets) {
  std::vector<const void *> in_ptrs;
  std::vector<void *> out_ptrs;
  for (size_t i = 0; i < args.size(); ++i) {
    auto buf = args.get<xla::ffi::AnyBuffer>(i);
    if (!buf.has_value()) return buf.error();
    in_ptrs.push_back(buf->untyped_data());
  }
  for (size_t i = 0; i < rets.size(); ++i) {
    auto buf = rets.get<xla::ffi::AnyBuffer>(i);
    if (!buf.has_value()) return buf.error();
    out_ptrs.push_back((*buf)->untyped_data());
  }
  std::string name(function_name);
  char *err = nullptr;
  int rc = ph_dispatch_device(hip_source.data(), hip_source.size(), name.c_str(),
                              grid_x, grid_y, grid_z, block_x, lanes, math_mode,
                              stream, in_ptrs.data(), in_ptrs.size(),
                              out_ptrs.data(), out_ptrs.size(), &err);
  if (rc != PH_OK) {
    std::string msg = err ? err : "ph_dispatch_device failed";
    ph_free_error(err);
    if (rc == PH_ERR_INVALID_ARGUMENT)
      return xla::ffi::Error::InvalidArgument(msg);
    return xla::ffi::Error::Internal(msg);
  }
  return xla::ffi::Error::Success();
}

}  // namespace

XLA_FFI_DEFINE_HANDLER_SYMBOL(palladium_hip_dispatch_rocm, PalladiumHipDispatchRocm,
                              xla::ffi::Ffi::Bind()
                                  .Ctx<xla::ffi::PlatformStream<hipStream_t>>()
                                  .Attr<std::string_view>("hip_source")
                                  .Attr<std::string_view>("function_name")
                                  .Attr<int64_t>("grid_x")
                                  .Attr<int64_t>("grid_y")
                                  .Attr<int64_t>("grid_z")
                                  .Attr<int64_t>("block_x")
                                  .Attr<int64_t>("lanes")
                                  .Attr<int64_t>("math_mode")
                                  .RemainingArgs()
                                  .RemainingRets());
