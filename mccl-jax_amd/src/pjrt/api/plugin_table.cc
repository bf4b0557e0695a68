// The exported entry point: GetPjrtApi() returns the process-lifetime
// PJRT_Api table (reference: pjrt_c_api.cc:877-884 and pjrt_c_api.h:6; the
// only symbol the library exports, per src/pjrt/api/exports.map).
//
// Every slot is filled from the slot list in pjrt_abi.h, so the table and
// the ABI cannot drift apart; the slots below with no implementation answer
// UNIMPLEMENTED "<slot> is not implemented in mi355x-pjrt".
#include <cstring>

#include "pjrt/api/plugin.h"

namespace mi::pjrt::slot {

#define MI_NOT_BUILT(X)                                                                       \
  X(CopyToDeviceStream_Destroy) X(CopyToDeviceStream_AddChunk) X(CopyToDeviceStream_TotalBytes) \
  X(CopyToDeviceStream_GranuleSize) X(CopyToDeviceStream_CurrentBytes) X(TopologyDescription_Serialize)

#define MI_REFUSE(Name)                                                                     \
  PJRT_Error* Name(PJRT_##Name##_Args*) {                                                   \
    return Fail(PJRT_Error_Code_UNIMPLEMENTED, "PJRT_" #Name " is not implemented in mi355x-pjrt"); \
  }
MI_NOT_BUILT(MI_REFUSE)
#undef MI_REFUSE

}  // namespace mi::pjrt::slot

extern "C" __attribute__((visibility("default"))) const PJRT_Api* GetPjrtApi() {
  static const PJRT_Api table = [] {
    PJRT_Api t;
    memset(&t, 0, sizeof(t));
    t.struct_size = sizeof(PJRT_Api);
    t.extension_start = nullptr;
    t.pjrt_api_version.struct_size = sizeof(PJRT_Api_Version);
    t.pjrt_api_version.major_version = MI_PJRT_API_MAJOR;
    t.pjrt_api_version.minor_version = MI_PJRT_API_MINOR;
#define MI_FILL(Name) t.PJRT_##Name = &mi::pjrt::slot::Name;
    MI_PJRT_SLOTS(MI_FILL, MI_FILL)
#undef MI_FILL
    return t;
  }();
  return &table;
}
