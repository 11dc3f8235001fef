// Kernel-choice table store (host code).
//
// The file follows the reference's tuning cache: `TORCHVULKAN_PIPELINE_CACHE=0`
// turns persistence off; the directory is $TORCHVULKAN_CACHE_DIR, else
// $XDG_CACHE_HOME/torchvulkan, else $HOME/.cache/torchvulkan
// (src/vulkan/cache.cpp:181-202); one file per device model. Each line is one
// result, `<format> <table> <key hex> <kernel id>`, appended in a single write
// so processes tuning at once interleave whole lines, and a later line wins
// (src/vulkan/autotuner.cpp:86-121). Lines of another format are skipped, as
// the reference skips results of another shader binary.
#include "tune_table.h"

#include <hip/hip_runtime.h>

#include <cctype>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <utility>

namespace tvk {
namespace {

constexpr const char* kFormat = "tvk1";

std::mutex g_mutex;
bool g_loaded = false;
std::string g_path;
std::map<std::pair<std::string, uint64_t>, std::string> g_table;

// gcnArchName up to its feature list, and the product name with blanks made '_'
std::string device_model() {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        (void)hipGetLastError();
        return "nodevice";
    }
    std::string arch = prop.gcnArchName;
    arch = arch.substr(0, arch.find(':'));
    std::string name = prop.name;
    for (char& c : name)
        if (!(std::isalnum(static_cast<unsigned char>(c)) || c == '-' || c == '.')) c = '_';
    return arch + "-" + name;
}

std::string cache_file() {
    const char* setting = std::getenv("TORCHVULKAN_PIPELINE_CACHE");
    if (setting != nullptr && std::strcmp(setting, "0") == 0) return {};
    std::filesystem::path dir;
    if (const char* custom = std::getenv("TORCHVULKAN_CACHE_DIR")) dir = custom;
    else if (const char* xdg = std::getenv("XDG_CACHE_HOME")) dir = std::filesystem::path(xdg) / "torchvulkan";
    else if (const char* home = std::getenv("HOME")) dir = std::filesystem::path(home) / ".cache" / "torchvulkan";
    else return {};
    return (dir / ("tuning-" + device_model() + ".txt")).string();
}

// caller holds g_mutex
void load_locked() {
    if (g_loaded) return;
    g_loaded = true;
    g_path = cache_file();
    if (g_path.empty()) return;
    std::ifstream file(g_path);
    std::string line;
    while (std::getline(file, line)) {
        std::istringstream fields(line);
        std::string format, kind, id;
        uint64_t key = 0;
        if (!(fields >> format >> kind >> std::hex >> key >> id) || format != kFormat) continue;
        g_table[{kind, key}] = id;
    }
}

}  // namespace

bool tune_lookup(const char* kind, uint64_t key, std::string& id) {
    std::lock_guard<std::mutex> lock(g_mutex);
    load_locked();
    auto it = g_table.find({kind, key});
    if (it == g_table.end()) return false;
    id = it->second;
    return true;
}

void tune_record(const char* kind, uint64_t key, const std::string& id, bool persist) {
    std::lock_guard<std::mutex> lock(g_mutex);
    load_locked();
    g_table[{kind, key}] = id;
    if (!persist || g_path.empty()) return;
    std::ostringstream line;
    line << kFormat << ' ' << kind << ' ' << std::hex << key << ' ' << id << '\n';
    std::error_code ec;
    std::filesystem::create_directories(std::filesystem::path(g_path).parent_path(), ec);
    std::ofstream(g_path, std::ios::app) << line.str() << std::flush;
}

void tune_reset() {
    std::lock_guard<std::mutex> lock(g_mutex);
    g_table.clear();
    g_loaded = false;
    g_path.clear();
}

std::string tune_path() {
    std::lock_guard<std::mutex> lock(g_mutex);
    load_locked();
    return g_path;
}

}  // namespace tvk
