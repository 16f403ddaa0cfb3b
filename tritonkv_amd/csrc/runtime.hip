// Device query and status text for the tritonkv_amd C ABI.
#include <hip/hip_runtime.h>
#include <string.h>

#include "../../include/tkv.h"

extern "C" int tkv_device_info(tkv_device_info_t* info) {
  if (!info) return TKV_EINVAL;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return TKV_ENODEVICE;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return (int)e;
  memset(info, 0, sizeof(*info));
  info->device = dev;
  info->compute_units = prop.multiProcessorCount;
  info->warp_size = prop.warpSize;
  info->l2_bytes = prop.l2CacheSize;
  info->global_mem_bytes = (int64_t)prop.totalGlobalMem;
  info->clock_khz = prop.clockRate;
  info->mem_clock_khz = prop.memoryClockRate;
  info->mem_bus_bits = prop.memoryBusWidth;
  strncpy(info->gcn_arch, prop.gcnArchName, sizeof(info->gcn_arch) - 1);
  return TKV_OK;
}

extern "C" const char* tkv_status_string(int status) {
  switch (status) {
    case TKV_OK: return "ok";
    case TKV_EINVAL: return "invalid argument";
    case TKV_EUNSUPPORTED: return "unsupported head_dim / nbits / group_size combination";
    case TKV_ENODEVICE: return "no HIP device";
    case TKV_ESCRATCH:
      return "split partials exceed the static scratch of tkv_fused_decode_attention_noalloc "
             "(TKV_NOALLOC_SCRATCH_BYTES)";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown tritonkv_amd status";
}

extern "C" int tkv_abi_version(void) { return 7; }
