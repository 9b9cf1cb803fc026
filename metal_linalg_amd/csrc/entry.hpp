// What every C entry point shares: the message of the calling thread's last
// failure (metal_linalg_last_error) and the mapping from an exception that
// escaped the library to a metal_linalg_status (std::invalid_argument ->
// INVALID_ARGUMENT, std::bad_alloc -> OUT_OF_MEMORY, anything else ->
// RUNTIME_ERROR), as the reference's C API reports them
// (reference: src/c_api.cpp:17-35).
#pragma once

#include <metal_linalg/c_api.h>

#include <exception>
#include <string>

namespace mla {

// This thread's last failure message ("" if none), kept until the next.
std::string& last_error_message();

// The status for the exception being handled; records its message.  Call
// only inside a catch block.
metal_linalg_status status_of_current_exception() noexcept;

// Runs `work`, returning OK or the status of what it threw.
template <class Work>
metal_linalg_status run_entry(Work&& work) noexcept {
    try {
        work();
        return METAL_LINALG_OK;
    } catch (...) {
        return status_of_current_exception();
    }
}

}  // namespace mla
