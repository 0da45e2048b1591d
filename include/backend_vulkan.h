/* backend_vulkan.h - lets c/qwen.c (#include "backend_vulkan.h", c/qwen.c:63-65) build
 * unchanged against libcoli_hip.so: the reference ABI is declared in coli_hip.h. */
#ifndef COLIBRI_BACKEND_VULKAN_H
#define COLIBRI_BACKEND_VULKAN_H
#include "coli_hip.h"
#endif
