# SPDX-License-Identifier: Apache-2.0
"""Static discovery manifest (data only; activates nothing)."""
