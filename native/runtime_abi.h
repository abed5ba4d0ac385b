/*
 * The runtime C-ABI header at the path the reference's native callers include it from
 * (native/runtime_abi_test.cpp:1 and native/runtime_api_client.cpp:1 include "runtime_abi.h"
 * from this directory, native/runtime_abi.h:1-9). A caller built with -I<repo>/native
 * compiles unchanged against libspaceslug_runtime.so. The declarations live in
 * include/runtime_abi.h.
 */
#ifndef SPACESLUG_NATIVE_RUNTIME_ABI_H
#define SPACESLUG_NATIVE_RUNTIME_ABI_H
#include "../include/runtime_abi.h"
#endif
