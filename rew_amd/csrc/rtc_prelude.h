// Included by vm_device.h when it is compiled by hipRTC for a generated
// kernel.  hipRTC has no libc headers; its fixed-width integer types live in
// __hip_internal.  Then the dtype codes of the public header.
#pragma once
typedef __hip_internal::int8_t int8_t;
typedef __hip_internal::uint8_t uint8_t;
typedef __hip_internal::int16_t int16_t;
typedef __hip_internal::uint16_t uint16_t;
typedef __hip_internal::int32_t int32_t;
typedef __hip_internal::uint32_t uint32_t;
typedef __hip_internal::int64_t int64_t;
typedef __hip_internal::uint64_t uint64_t;
// the public header, registered with hipRTC under this plain name
#include "rew_mi355x.h"
