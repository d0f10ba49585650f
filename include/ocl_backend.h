/* SPDX-License-Identifier: Unlicense */

/* The name the reference's sources include (main.c:38, ops.h:6,
 * disk.h:6 of i.coregistration.opencl): the backend is the HIP one. */

#ifndef ICOREG_OCL_BACKEND_H
#define ICOREG_OCL_BACKEND_H

#include "hip_backend.h"

#endif /* ICOREG_OCL_BACKEND_H */
