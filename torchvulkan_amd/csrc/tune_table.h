// Kernel-choice table: shape class -> the kernel chosen for it, kept in
// memory and persisted one line per result in the tuning file.
//
// Reference: Autotuner::select/load/save (src/vulkan/autotuner.cpp:56-121)
// and the cache file location (VulkanCache::cachePath,
// src/vulkan/cache.cpp:181-202).
#pragma once

#include <cstdint>
#include <string>

namespace tvk {

// The choice recorded for `key` in table `kind` ("gemm"); the tuning file is
// read on first use. False when there is none.
bool tune_lookup(const char* kind, uint64_t key, std::string& id);

// Records a choice (a later record of the same key wins) and, with persist,
// appends it to the tuning file.
void tune_record(const char* kind, uint64_t key, const std::string& id, bool persist);

// Forgets every choice; the next lookup reads the environment and the file again.
void tune_reset();

// The tuning file in use ("" when persistence is off).
std::string tune_path();

}  // namespace tvk
