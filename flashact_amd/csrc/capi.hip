// Library-wide C-ABI entry points: error text, ABI version, device query, launch checks.
#include <mutex>
#include <string.h>

#include "../../include/flashact_mi355x.h"
#include "fa_host.h"

namespace fa {
namespace host {

char* error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}

namespace {
struct DevState {
  bool probed = false;
  hipDeviceProp_t prop;
  int coop = 0;
};
std::mutex g_mu;
DevState g_dev[64];
struct KernelAttr {
  const void* kernel;
  int device;
  unsigned lds;
};
KernelAttr g_attr[64];
int g_nattr = 0;
}  // namespace

int check_device(const void* kernel, int threads, unsigned lds_bytes, int nwg, const char* who) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FA_ERR_DEVICE, "%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(FA_ERR_DEVICE, "%s: device ordinal %d out of range", who, dev);
  std::lock_guard<std::mutex> lk(g_mu);
  DevState& d = g_dev[dev];
  if (!d.probed) {
    e = hipGetDeviceProperties(&d.prop, dev);
    if (e != hipSuccess) return fail(FA_ERR_DEVICE, "%s: hipGetDeviceProperties: %s", who, hipGetErrorString(e));
    if (hipDeviceGetAttribute(&d.coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) d.coop = 0;
    d.probed = true;
  }
  if (strncmp(d.prop.gcnArchName, "gfx950", 6) != 0)
    return fail(FA_ERR_DEVICE, "%s: device %d is %s; this library is built for gfx950 (MI355X)", who, dev,
                d.prop.gcnArchName);
  if (d.prop.multiProcessorCount != 256)
    return fail(FA_ERR_DEVICE, "%s: device %d has %d CUs; the XCD-aware schedule needs 256 (8 XCDs x 32)", who, dev,
                d.prop.multiProcessorCount);
  if (!d.coop) return fail(FA_ERR_DEVICE, "%s: device %d does not support cooperative launch", who, dev);
  bool have = false;
  for (int i = 0; i < g_nattr; i++)
    if (g_attr[i].kernel == kernel && g_attr[i].device == dev && g_attr[i].lds == lds_bytes) have = true;
  if (!have) {
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
    if (e != hipSuccess) return fail(FA_ERR_DEVICE, "%s: hipFuncSetAttribute(LDS=%u): %s", who, lds_bytes,
                                     hipGetErrorString(e));
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds_bytes);
    if (e != hipSuccess) return fail(FA_ERR_DEVICE, "%s: occupancy query: %s", who, hipGetErrorString(e));
    if (per_cu * d.prop.multiProcessorCount < nwg)
      return fail(FA_ERR_DEVICE, "%s: only %d x %d workgroups can be co-resident, need %d", who, per_cu,
                  d.prop.multiProcessorCount, nwg);
    if (g_nattr < 64) g_attr[g_nattr++] = KernelAttr{kernel, dev, lds_bytes};
  }
  return FA_OK;
}

int coop_launch(const void* kernel, int nwg, int threads, void** args, unsigned lds, fa_stream_t stream,
                const char* who) {
  const hipError_t e =
      hipLaunchCooperativeKernel(kernel, dim3(nwg), dim3(threads), args, lds, (hipStream_t)stream);
  if (e == hipSuccess) return FA_OK;
  if (e == hipErrorIllegalState)
    return fail(FA_ERR_LAUNCH,
                "%s: the runtime refused the cooperative launch (%s). This happens in a process whose parent "
                "had already made a cooperative launch when it started this one: start worker processes before "
                "the parent's first launch (or from a parent that never launches)",
                who, hipGetErrorString(e));
  return fail(FA_ERR_LAUNCH, "%s: cooperative launch failed: %s", who, hipGetErrorString(e));
}

}  // namespace host
}  // namespace fa

extern "C" const char* fa_last_error(void) { return fa::host::error_buffer(); }

extern "C" int fa_abi_version(void) { return FA_ABI_VERSION; }

extern "C" int fa_device_query(int device, fa_device_info* info) {
  if (!info) return fa::host::fail(FA_ERR_INVALID_ARG, "fa_device_query: info is NULL");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fa::host::fail(FA_ERR_DEVICE, "fa_device_query: %s", hipGetErrorString(e));
  memset(info, 0, sizeof(*info));
  info->cus = prop.multiProcessorCount;
  info->xcds = prop.multiProcessorCount / 32;
  info->lds_bytes = (int)prop.sharedMemPerBlock;
  if (hipDeviceGetAttribute(&info->coop_launch, hipDeviceAttributeCooperativeLaunch, device) != hipSuccess)
    info->coop_launch = 0;
  info->coop_max_blocks = fa::pi05_bs1_coop_capacity(device);
  strncpy(info->arch, prop.gcnArchName, sizeof(info->arch) - 1);
  return FA_OK;
}
