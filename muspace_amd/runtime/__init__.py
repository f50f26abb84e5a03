"""Native loader and dispatch reporting for the MSDA operator."""
